// Lane reductions through DPP moves (no LDS round trips), shared by the
// kernel files.
#pragma once

#include <hip/hip_runtime.h>

namespace meshgpt::kern {

// v moved by the DPP pattern CTRL; lanes the pattern gives no source keep `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_move(float old, float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                 0xf, false));
}

// Sum over the wave: quad swaps, half-row and row mirrors, then the row
// broadcasts of GFX9; the total lands in lane 63 and is read back to every
// lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_move<0xB1>(0.0f, v);       // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(0.0f, v);       // quad_perm [2,3,0,1]
    v += dpp_move<0x141>(0.0f, v);      // row_half_mirror
    v += dpp_move<0x140>(0.0f, v);      // row_mirror
    v += dpp_move<0x142, 0xa>(0.0f, v); // row_bcast:15
    v += dpp_move<0x143, 0xc>(0.0f, v); // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Sum over aligned groups of N lanes (N a power of two <= 64), left in every
// lane of the group: DPP quad swaps and row mirrors inside a 16-lane row, then
// lane shuffles across rows.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) v += dpp_move<0xB1>(0.0f, v);   // quad_perm [1,0,3,2]
    if constexpr (N >= 4) v += dpp_move<0x4E>(0.0f, v);   // quad_perm [2,3,0,1]
    if constexpr (N >= 8) v += dpp_move<0x141>(0.0f, v);  // row_half_mirror
    if constexpr (N >= 16) v += dpp_move<0x140>(0.0f, v); // row_mirror
    if constexpr (N >= 32) v += __shfl_xor(v, 16, 64);
    if constexpr (N >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

}  // namespace meshgpt::kern
