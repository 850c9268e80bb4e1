// Device helpers shared by the attention kernels.
#pragma once
#include "common.h"
#include <type_traits>

// Combine a lane's value with the same lane position of the other 32-lane half.
__device__ inline float half_max(float x) { return fmaxf(x, __shfl_xor(x, 32, 64)); }
__device__ inline float half_sum(float x) { return x + __shfl_xor(x, 32, 64); }

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ inline float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }
