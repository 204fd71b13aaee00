// Shared helpers for libgphq: error codes, launch checks, wavefront reductions.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "../../include/gphq.h"

namespace gphq {

// Records the most recent HIP failure so gphq_last_hip_error() can report it.
void set_hip_error(hipError_t e);

// Converts a HIP status into a gphq status, remembering the HIP code.
inline int hip_status(hipError_t e) {
    if (e == hipSuccess) return GPHQ_OK;
    set_hip_error(e);
    return GPHQ_ERR_HIP;
}

// Checks the launch that was just enqueued.
inline int launch_status() { return hip_status(hipGetLastError()); }

#define GPHQ_TRY(expr)                      \
    do {                                    \
        int _st = (expr);                   \
        if (_st != GPHQ_OK) return _st;     \
    } while (0)

// ---- device helpers --------------------------------------------------------

// Butterfly sum inside each row of 16 lanes, using DPP lane permutes, so every
// lane of a row ends with that row's total. quad_perm [1,0,3,2] and [2,3,0,1]
// pair lanes at distance 1 and 2; row_half_mirror pairs the two quads of an
// 8-lane half; row_mirror pairs the two halves of a row.
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    return v;
}

// Sum over the 64 lanes of a wavefront; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (a + b) + (c + d);
}

// IEEE half bits -> float (exact), for FP16 scales stored as raw uint16.
__device__ __forceinline__ float half_bits_to_float(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

}  // namespace gphq
