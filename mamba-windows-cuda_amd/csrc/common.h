// Shared device/host helpers for the gfx950 selective-scan kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mwc_ssm.h"

namespace mwc {

constexpr int kNState = 16;          // the reference's N_STATE (mamba_cuda.py:62)
constexpr int kCkptSteps = MWC_CKPT_STEPS;
constexpr float kLog2e = 1.4426950408889634f;
// safe_exp clamps delta*A to [-88, 88] (mamba_cuda.py:65-70); in base 2 that is +-88*log2(e).
constexpr float kExp2Clamp = 88.0f * 1.4426950408889634f;

typedef _Float16 half_t;

template <typename T> __device__ __forceinline__ float ld(const T* p) { return static_cast<float>(*p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v) { *p = static_cast<T>(v); }

// exp(x) for x = delta*A given x2 = x*log2(e): clamp then the hardware base-2 exponential.
__device__ __forceinline__ float exp2_clamped(float x2) {
    return __builtin_amdgcn_exp2f(__builtin_fminf(__builtin_fmaxf(x2, -kExp2Clamp), kExp2Clamp));
}

// DPP lane exchanges within 16-lane rows (gfx9 DPP controls).
template <int CTRL> __device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within each 16

// All-reduce (sum) over aligned groups of G consecutive lanes, G in {1,2,4,8,16}.
// After the quad steps every lane of a quad holds the quad sum, so the mirror
// exchanges (which pair lanes of different quads / halves) complete the sum.
template <int G> __device__ __forceinline__ float group_sum(float v) {
    if constexpr (G >= 2) v += dpp<kDppXor1>(v);
    if constexpr (G >= 4) v += dpp<kDppXor2>(v);
    if constexpr (G >= 8) v += dpp<kDppHalfMirror>(v);
    if constexpr (G >= 16) v += dpp<kDppMirror>(v);
    return v;
}

}  // namespace mwc

#define MWC_HIP_TRY(expr)                                  \
    do {                                                   \
        hipError_t _e = (expr);                            \
        if (_e != hipSuccess) return mwc_set_hip_error(_e, #expr); \
    } while (0)

int mwc_set_error(int status, const char* msg);
int mwc_set_hip_error(hipError_t e, const char* what);
