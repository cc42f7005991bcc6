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

// Value of lane ^ 16: v_permlane16_swap of v with itself trades odd rows of
// the first operand with even rows of the second, so result [1] holds row
// r ^ 1 in even rows and [0] in odd rows (a VALU exchange, no LDS).
__device__ __forceinline__ float row_swap(float v, bool odd_row) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, odd_row ? r[0] : r[1]);
}

// Transpose-sum inside aligned groups of G lanes (G = 4, 8, 16 or 32), each
// lane holding G values: afterwards lane l holds the group's total of value
// index l % G.  Each stage halves the values a lane carries -- a lane keeps
// the upper half when its stage bit is set and adds the partner's copy of
// the half it keeps -- so the cost is G - 1 exchanges instead of G full
// reductions.  Partners: lane ^ 16 (row swap), then row mirror, half-row
// mirror, quad swaps (DPP); a mirror partner differs in the stage bit and
// shares every higher bit, which is all the pairing needs.
template <int CTRL, int N>
__device__ __forceinline__ void transpose_stage(float *v, bool upper) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const float send = upper ? v[i] : v[i + N];
        const float keep = upper ? v[i + N] : v[i];
        if constexpr (CTRL < 0) v[i] = keep + row_swap(send, upper);
        else v[i] = keep + dpp<CTRL>(send);
    }
}

template <int G>
__device__ __forceinline__ float transpose_sum(float (&v)[G], int lane) {
    static_assert(G == 4 || G == 8 || G == 16 || G == 32, "group of 4, 8, 16 or 32 lanes");
    if constexpr (G >= 32) transpose_stage<-1, 16>(v, lane & 16);
    if constexpr (G >= 16) transpose_stage<kRowMirror, 8>(v, lane & 8);
    if constexpr (G >= 8) transpose_stage<kHalfMirror, 4>(v, lane & 4);
    transpose_stage<kXor2, 2>(v, lane & 2);
    transpose_stage<kXor1, 1>(v, lane & 1);
    return v[0];
}

}  // namespace wave
}  // namespace tbh
