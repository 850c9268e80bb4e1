// Device helpers shared by the attention kernels.
#pragma once
#include "common.h"
#include <type_traits>

// Combine a lane's value with the same lane position of the other 32-lane half.
__device__ inline float half_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
__device__ inline float half_sum(float x) { return x + __shfl_xor(x, 32, 64); }

// The same on the VALU without an LDS round trip: v_permlane32_swap of x with
// itself leaves the low half's values in one result and the high half's in the
// other (in every lane), so their max / sum is the combination.
__device__ inline float half_max_swap(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ inline float half_sum_swap(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ inline float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }
