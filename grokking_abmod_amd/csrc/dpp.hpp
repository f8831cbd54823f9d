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

// wave_sum of eight values at once: lane l returns the sum over the wave of
// v[l & 7].  The lanes add the same pairs level by level as wave_sum does
// (lane bits 0, 1, 2, 3, 4, 5), and f32 addition is commutative, so every
// sum is wave_sum's bit for bit.  At each of the first three levels a lane
// keeps one value of each pair of rows and sends the other to its partner,
// which keeps that one, so the values a lane holds halve: 10 adds instead of
// 48, and no dependent chain of six DPP steps per row.
__device__ __forceinline__ float wave_sum8(const float (&v)[8], int lane) {
    const bool b0 = lane & 1, b1 = lane & 2, b2 = lane & 4;
    float a[4], b[2];
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // lane ^ 1: a[k] holds row 2k + b0
        const float keep = b0 ? v[2 * k + 1] : v[2 * k], send = b0 ? v[2 * k] : v[2 * k + 1];
        a[k] = keep + dpp_move<0xB1>(0.0f, send);  // quad_perm [1,0,3,2]
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // lane ^ 2: b[k] holds row 4k + 2 b1 + b0
        const float keep = b1 ? a[2 * k + 1] : a[2 * k], send = b1 ? a[2 * k] : a[2 * k + 1];
        b[k] = keep + dpp_move<0x4E>(0.0f, send);  // quad_perm [2,3,0,1]
    }
    // lane ^ 4: lanes with bit 2 set read 4 lanes down (row_ror:4), the
    // others 4 lanes up (row_ror:12); c holds row l & 7.
    const float keep = b2 ? b[1] : b[0], send = b2 ? b[0] : b[1];
    const float down = dpp_move<0x124>(0.0f, send), up = dpp_move<0x12C>(0.0f, send);
    float c = keep + (b2 ? down : up);
    c += dpp_move<0x128>(0.0f, c);  // lane ^ 8: row_ror:8
    // lane ^ 16 and lane ^ 32: each swap leaves the two rows (halves) to be
    // added in its two results.
    const auto s = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, c), __builtin_bit_cast(int, c),
                                                    false, false);
    c = __builtin_bit_cast(float, int(s[0])) + __builtin_bit_cast(float, int(s[1]));
    const auto t = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, c), __builtin_bit_cast(int, c),
                                                    false, false);
    return __builtin_bit_cast(float, int(t[0])) + __builtin_bit_cast(float, int(t[1]));
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
