// Device helpers shared by the attention kernels.
#pragma once
#include "common.h"

// Value held by the same lane position in the other 32-lane half of the wavefront.
__device__ inline float half_swap(float x) { return __shfl_xor(x, 32, 64); }

// 2^x on the transcendental unit (v_exp_f32); exp2(-inf) = 0.
__device__ inline float exp2f_fast(float x) { return __builtin_amdgcn_exp2f(x); }
