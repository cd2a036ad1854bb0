// Shared device/host helpers for the gfx950 selective-scan kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mwc_ssm.h"

namespace mwc {

constexpr int kCkptSteps = MWC_CKPT_STEPS;
constexpr float kLog2e = 1.4426950408889634f;
// safe_exp clamps delta*A to [-88, 88] (mamba_cuda.py:65-70); in base 2 that is +-88*log2(e).
constexpr float kExp2Clamp = 88.0f * 1.4426950408889634f;

typedef _Float16 half_t;
typedef __bf16 bf16_t;  // storage only: converted to fp32 on load, rounded to nearest even on store

// Storage dtype codes (mwc_dtype) and a dispatcher over the storage type.
#define MWC_DISPATCH_DTYPE(dt, TT, ...)              \
    do {                                               \
        if ((dt) == MWC_DTYPE_F16) {                   \
            typedef half_t TT;                         \
            __VA_ARGS__;                               \
        } else if ((dt) == MWC_DTYPE_BF16) {           \
            typedef bf16_t TT;                         \
            __VA_ARGS__;                               \
        } else {                                       \
            typedef float TT;                          \
            __VA_ARGS__;                               \
        }                                              \
    } while (0)

template <typename T> __device__ __forceinline__ float ld(const T* p) { return static_cast<float>(*p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v) { *p = static_cast<T>(v); }

// exp(x) for x = delta*A given x2 = x*log2(e): clamp then the hardware base-2 exponential.
__device__ __forceinline__ float exp2_clamped(float x2) {
    return __builtin_amdgcn_exp2f(__builtin_fminf(__builtin_fmaxf(x2, -kExp2Clamp), kExp2Clamp));
}

// Raw buffer access (gfx9 buffer resource, stride 0): a load whose byte offset is at or beyond the
// resource's size returns 0 and such a store is dropped, so tails and padding lanes need no branches.
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 dword 3: 32-bit data format, no swizzle
constexpr uint32_t kOob = 0x80000000u;   // an offset past every resource built here (sizes < 2^31)
typedef __amdgpu_buffer_rsrc_t rsrc_t;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}
template <typename T> __device__ __forceinline__ float buf_ld(rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ float buf_ld<float>(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
template <> __device__ __forceinline__ float buf_ld<half_t>(rsrc_t r, uint32_t off) {
    return static_cast<float>(__builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)));
}
template <> __device__ __forceinline__ float buf_ld<bf16_t>(rsrc_t r, uint32_t off) {
    return static_cast<float>(__builtin_bit_cast(bf16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)));
}
// Raw storage-type load (conversion deferred, keeps fp16 values in 16 bits while in flight).
template <typename T> __device__ __forceinline__ T buf_raw(rsrc_t r, uint32_t off);
template <> __device__ __forceinline__ float buf_raw<float>(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
template <> __device__ __forceinline__ half_t buf_raw<half_t>(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(half_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <> __device__ __forceinline__ bf16_t buf_raw<bf16_t>(rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(bf16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
}
template <typename T> __device__ __forceinline__ void buf_st(rsrc_t r, uint32_t off, float v);
template <> __device__ __forceinline__ void buf_st<float>(rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v), r, off, 0, 0);
}
template <> __device__ __forceinline__ void buf_st<half_t>(rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(short, static_cast<half_t>(v)), r, off, 0, 0);
}
template <> __device__ __forceinline__ void buf_st<bf16_t>(rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(short, static_cast<bf16_t>(v)), r, off, 0, 0);
}
// K consecutive fp32 values (K = 1, 2 or a multiple of 4) as 4-, 8- or 16-byte buffer stores.
template <int K> __device__ __forceinline__ void buf_st_f32(rsrc_t r, uint32_t off, const float (&v)[K]) {
    typedef int v2i __attribute__((ext_vector_type(2)));
    typedef int v4i __attribute__((ext_vector_type(4)));
    if constexpr (K == 1) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(int, v[0]), r, off, 0, 0);
    } else if constexpr (K == 2) {
        const v2i q = {__builtin_bit_cast(int, v[0]), __builtin_bit_cast(int, v[1])};
        __builtin_amdgcn_raw_buffer_store_b64(q, r, off, 0, 0);
    } else {
        static_assert(K % 4 == 0, "vector width");
#pragma unroll
        for (int k = 0; k < K; k += 4) {
            const v4i q = {__builtin_bit_cast(int, v[k]), __builtin_bit_cast(int, v[k + 1]),
                           __builtin_bit_cast(int, v[k + 2]), __builtin_bit_cast(int, v[k + 3])};
            __builtin_amdgcn_raw_buffer_store_b128(q, r, off + 4 * k, 0, 0);
        }
    }
}

// Issue priority by progress through a workgroup's chunks. A SIMD's arbiter issues from the
// highest-priority ready wave and, among equals, from the oldest, so workgroups that share a CU and
// start together would finish in dispatch order, far apart (the fused backward at 3 workgroups per
// CU: 210, 253 and 302 us), and the last would run alone at a fraction of the CU's throughput.
// Dropping a wave's priority as it passes 1/2, 3/4 and 7/8 of its chunks lets the ones behind
// catch up, so they finish close together.
struct ProgressPrio {
    int b1, b2, b3;  // chunks done at which the priority drops to 2, 1, 0
    __device__ __forceinline__ explicit ProgressPrio(int nchunks)
        : b1(nchunks / 2), b2(3 * nchunks / 4), b3(7 * nchunks / 8) {
        __builtin_amdgcn_s_setprio(3);
    }
    __device__ __forceinline__ void update(int done) {
        if (done == b1 || done == b2 || done == b3) {
            if (done == b3)
                __builtin_amdgcn_s_setprio(0);
            else if (done == b2)
                __builtin_amdgcn_s_setprio(1);
            else
                __builtin_amdgcn_s_setprio(2);
        }
    }
};

// Elementwise transforms around the scan, from the hardware base-2 exp/log and reciprocal
// (each ~1 ulp). softplus(x) = ln(1 + e^x): x itself above 20 (as torch's threshold), the series
// t - t^2/2 + t^3/3 for t = e^x < 2^-6 (where 1 + t would round away t's low bits; the first
// omitted term is below 2^-20 relative), else ln2 * log2(1 + t).
constexpr float kLn2 = 0.6931471805599453f;
// Both forms are computed and then selected, so the code is straight-line rather than a divergent
// branch; the unselected form may be inf or NaN above the threshold, and a NaN x stays NaN.
__device__ __forceinline__ float softplus_f(float x) {
    const float t = __builtin_amdgcn_exp2f(x * kLog2e);
    float series = t * __builtin_fmaf(t, __builtin_fmaf(t, 1.f / 3.f, -0.5f), 1.f);
    float big = kLn2 * __builtin_amdgcn_logf(1.f + t);
    asm("" : "+v"(series), "+v"(big));
    return x > 20.f ? x : (t < 0.015625f ? series : big);
}
__device__ __forceinline__ float sigmoid_f(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}
// softplus(x) and its derivative sigmoid(x) = t / (1 + t), sharing the one exponential t = e^x;
// above the threshold sigmoid(x) is 1 in fp32
__device__ __forceinline__ float softplus_grad_f(float x, float& sig) {
    const float t = __builtin_amdgcn_exp2f(x * kLog2e);
    const float u = 1.f + t;
    float s = t * __builtin_amdgcn_rcpf(u);
    float series = t * __builtin_fmaf(t, __builtin_fmaf(t, 1.f / 3.f, -0.5f), 1.f);
    float big = kLn2 * __builtin_amdgcn_logf(u);
    asm("" : "+v"(series), "+v"(big), "+v"(s));
    const bool above = x > 20.f;
    sig = above ? 1.f : s;
    return above ? x : (t < 0.015625f ? series : big);
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

// Reduce-scatter over aligned groups of G lanes (G in {2,4,8,16}) of V values per lane (V a power of
// two, 2 <= V <= G): the lane returns the group sum of value rs_index<G, V>(lane); each index is held
// by G/V lanes of the group. The levels pair a lane with its DPP partner, first across the 4-lane
// banks of the 16-lane row (mirror in 16, then mirror in 8), then inside a bank (xor 2, xor 1). At the
// first log2(V) levels the pair splits its values by a lane bit that differs between the partners and
// agrees on every earlier level's bit -- i3, i2, i1, i0 of the lane's index i in its row, in that
// level order -- each lane keeping one half and adding the partner's copy of it; the remaining levels
// add the single value. Across banks the bit is a function of the bank, so one DPP add per half, each
// enabled on the banks that keep that half, does a pair in two instructions; inside a bank it takes
// two selects and one DPP add.
template <int G> __device__ __forceinline__ int rs_bit(int level, int lane) {
    // level order: mirror in 16 (G = 16 only), mirror in 8 (G >= 8), xor 2 (G >= 4), xor 1
    constexpr int first = G >= 16 ? 3 : G >= 8 ? 2 : G >= 4 ? 1 : 0;  // lane bit of level 0
    return (lane >> (first - level)) & 1;
}
template <int G, int V> __device__ __forceinline__ int rs_index(int lane) {
    int idx = 0;
#pragma unroll
    for (int l = 0; (1 << l) < V; ++l) idx |= rs_bit<G>(l, lane) << l;
    return idx;
}
// The partner's copy of v at the level whose partner flips lane bits 0..b (b = 3: mirror in 16,
// b = 2: mirror in 8, b = 1: xor 2, b = 0: xor 1).
template <int B> __device__ __forceinline__ float dpp_flip(float v) {
    if constexpr (B == 3) return dpp<kDppMirror>(v);
    if constexpr (B == 2) return dpp<kDppHalfMirror>(v);
    if constexpr (B == 1) return dpp<kDppXor2>(v);
    if constexpr (B == 0) return dpp<kDppXor1>(v);
}
// One cross-bank level of the reduce-scatter on NP value pairs: lanes whose bank keeps half 0 get
// x[2q] + the partner's x[2q], the others x[2q+1] + the partner's x[2q+1]. B = 3: mirror in 16, lane bit
// i3 (banks 0,1 keep half 0); B = 2: mirror in 8, lane bit i2 (banks 0,2). Each pair is two DPP adds,
// each enabled on the banks that keep its half. The leading s_nop gives the two wait states a DPP read
// needs after a VALU write of its source; the trailing one covers a DPP read of the results after the
// block (the compiler does not look inside it).
template <int B, int NP> __device__ __forceinline__ void dpp_bank_level(const float* x, float* r);

// DPP controls and bank masks (half 0, half 1) of the two cross-bank levels
#define MWC_BANK_ADD(o, i0, i1, ctrl, m0, m1)                                   \
    "v_add_f32_dpp %" #o ", %" #i0 ", %" #i0 " " ctrl " row_mask:0xf bank_mask:" m0 "\n\t" \
    "v_add_f32_dpp %" #o ", %" #i1 ", %" #i1 " " ctrl " row_mask:0xf bank_mask:" m1 "\n\t"
#define MWC_BANK_LEVEL(B, CTRL, M0, M1)                                                                    \
    template <> __device__ __forceinline__ void dpp_bank_level<B, 1>(const float* x, float* r) {            \
        asm("s_nop 1\n\t" MWC_BANK_ADD(0, 1, 2, CTRL, M0, M1) "s_nop 1"                                      \
            : "=&v"(r[0])                                                                                  \
            : "v"(x[0]), "v"(x[1]));                                                                       \
    }                                                                                                      \
    template <> __device__ __forceinline__ void dpp_bank_level<B, 2>(const float* x, float* r) {            \
        asm("s_nop 1\n\t" MWC_BANK_ADD(0, 2, 3, CTRL, M0, M1) MWC_BANK_ADD(1, 4, 5, CTRL, M0, M1) "s_nop 1"   \
            : "=&v"(r[0]), "=&v"(r[1])                                                                     \
            : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));                                                 \
    }                                                                                                      \
    template <> __device__ __forceinline__ void dpp_bank_level<B, 4>(const float* x, float* r) {            \
        asm("s_nop 1\n\t" MWC_BANK_ADD(0, 4, 5, CTRL, M0, M1) MWC_BANK_ADD(1, 6, 7, CTRL, M0, M1)           \
                MWC_BANK_ADD(2, 8, 9, CTRL, M0, M1) MWC_BANK_ADD(3, 10, 11, CTRL, M0, M1) "s_nop 1"          \
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])                                           \
            : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]));     \
    }                                                                                                      \
    template <> __device__ __forceinline__ void dpp_bank_level<B, 8>(const float* x, float* r) {            \
        asm("s_nop 1\n\t" MWC_BANK_ADD(0, 8, 9, CTRL, M0, M1) MWC_BANK_ADD(1, 10, 11, CTRL, M0, M1)         \
                MWC_BANK_ADD(2, 12, 13, CTRL, M0, M1) MWC_BANK_ADD(3, 14, 15, CTRL, M0, M1)                  \
                MWC_BANK_ADD(4, 16, 17, CTRL, M0, M1) MWC_BANK_ADD(5, 18, 19, CTRL, M0, M1)                  \
                MWC_BANK_ADD(6, 20, 21, CTRL, M0, M1) MWC_BANK_ADD(7, 22, 23, CTRL, M0, M1) "s_nop 1"        \
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4]), "=&v"(r[5]), "=&v"(r[6]),   \
              "=&v"(r[7])                                                                                  \
            : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]),      \
              "v"(x[8]), "v"(x[9]), "v"(x[10]), "v"(x[11]), "v"(x[12]), "v"(x[13]), "v"(x[14]),            \
              "v"(x[15]));                                                                                 \
    }
MWC_BANK_LEVEL(3, "row_mirror", "0x3", "0xc")       // lane bit i3: banks 0,1 keep half 0
MWC_BANK_LEVEL(2, "row_half_mirror", "0x5", "0xa")  // lane bit i2: banks 0,2 keep half 0
#undef MWC_BANK_LEVEL
#undef MWC_BANK_ADD

template <int G, int V, int L = 0, int M = V>
__device__ __forceinline__ float reduce_scatter_lv(float (&x)[V], int lane) {
    static_assert(V >= 2 && V <= G && (V & (V - 1)) == 0 && (G & (G - 1)) == 0 && G <= 16, "shape");
    constexpr int first = G >= 16 ? 3 : G >= 8 ? 2 : G >= 4 ? 1 : 0;
    constexpr int B = first - L;  // lane bit (and partner) of this level
    if constexpr (B < 0) {
        return x[0];
    } else if constexpr (M > 1) {
        if constexpr (B >= 2) {
            float r[M / 2];
            dpp_bank_level<B, M / 2>(x, r);
#pragma unroll
            for (int q = 0; q < M / 2; ++q) x[q] = r[q];
        } else {
            const bool hi = rs_bit<G>(L, lane) != 0;
#pragma unroll
            for (int q = 0; q < M / 2; ++q) {
                const float keep = hi ? x[2 * q + 1] : x[2 * q];
                const float send = hi ? x[2 * q] : x[2 * q + 1];
                x[q] = keep + dpp_flip<B>(send);
            }
        }
        return reduce_scatter_lv<G, V, L + 1, M / 2>(x, lane);
    } else {
        x[0] += dpp_flip<B>(x[0]);
        return reduce_scatter_lv<G, V, L + 1, 1>(x, lane);
    }
}
// x is clobbered.
template <int G, int V> __device__ __forceinline__ float reduce_scatter(float (&x)[V], int lane) {
    return reduce_scatter_lv<G, V>(x, lane);
}

// Reduce-scatter over the LPC = 64/CPW lanes of a channel when the wave's CPW channels occupy the
// low lane bits (channel = lane % CPW, state group = lane / CPW): the partners of a channel's lanes
// differ in lane bits log2(CPW)..5, and every such bit has a two-instruction exchange on gfx950 --
// bits 4 and 5 swap rows / halves of a register pair (v_permlane16_swap_b32, v_permlane32_swap_b32),
// bits 3 and 2 are DPP reads of lane +-8 / +-4 whose halves are selected by bank masks. So each level
// costs two instructions per value it leaves (no selects), and a last single-value level on a DPP bit
// costs one. Level order: the permlane bits first (while two or more values remain), then bits 3, 2.
// At a level on lane bit b the lanes with bit b = 0 keep the even values (2q) and the others the odd
// ones (2q+1), each adding its partner's copy; the lane returns the group sum of value
// rs_hi_index<CPW, V>(lane). The clang builtins for the permlane swaps drop their second result in this
// toolchain, so they are written as inline assembly with both registers read and written; a leading
// s_nop covers the read-after-VALU-write wait states of DPP and permlane sources.
template <int CPW> constexpr int hi_log() { return CPW >= 16 ? 4 : CPW >= 8 ? 3 : CPW >= 4 ? 2 : CPW >= 2 ? 1 : 0; }
template <int CPW> constexpr int hi_bit(int level) {
    constexpr int order[6] = {4, 5, 3, 2, 1, 0};
    int k = 0;
    for (int i = 0; i < 6; ++i)
        if (order[i] >= hi_log<CPW>()) {
            if (k == level) return order[i];
            ++k;
        }
    return -1;
}
template <int CPW, int V> __device__ __forceinline__ int rs_hi_index(int lane) {
    int idx = 0;
#pragma unroll
    for (int l = 0; (1 << l) < V; ++l) idx |= ((lane >> hi_bit<CPW>(l)) & 1) << l;
    return idx;
}

// v_permlane{16,32}_swap_b32 on NP register pairs (x[2q], x[2q+1]), in place
template <int BIT, int NP> __device__ __forceinline__ void permlane_swap_pairs(float* x);
#define MWC_PL(BIT, INS)                                                                                       \
    template <> __device__ __forceinline__ void permlane_swap_pairs<BIT, 1>(float* x) {                        \
        asm("s_nop 1\n\t" INS " %0, %1" : "+v"(x[0]), "+v"(x[1]));                                              \
    }                                                                                                          \
    template <> __device__ __forceinline__ void permlane_swap_pairs<BIT, 2>(float* x) {                        \
        asm("s_nop 1\n\t" INS " %0, %1\n\t" INS " %2, %3" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));  \
    }                                                                                                          \
    template <> __device__ __forceinline__ void permlane_swap_pairs<BIT, 4>(float* x) {                        \
        asm("s_nop 1\n\t" INS " %0, %1\n\t" INS " %2, %3\n\t" INS " %4, %5\n\t" INS " %6, %7"                  \
            : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7])); \
    }                                                                                                          \
    template <> __device__ __forceinline__ void permlane_swap_pairs<BIT, 8>(float* x) {                        \
        permlane_swap_pairs<BIT, 4>(x);                                                                        \
        permlane_swap_pairs<BIT, 4>(x + 8);                                                                    \
    }
MWC_PL(4, "v_permlane16_swap_b32")
MWC_PL(5, "v_permlane32_swap_b32")
#undef MWC_PL

// DPP levels on lane bit 3 (partner lane ^ 8: row_ror:8; banks 0,1 keep half 0) and bit 2 (partner
// lane + 4 on banks 0,2 via row_shl:4, lane - 4 on banks 1,3 via row_shr:4; banks 0,2 keep half 0)
#define MWC_HADD(o, i0, i1, c0, c1, m0, m1)                                                          \
    "v_add_f32_dpp %" #o ", %" #i0 ", %" #i0 " " c0 " row_mask:0xf bank_mask:" m0 "\n\t"              \
    "v_add_f32_dpp %" #o ", %" #i1 ", %" #i1 " " c1 " row_mask:0xf bank_mask:" m1 "\n\t"
template <int BIT, int NP> __device__ __forceinline__ void dpp_hi_level(const float* x, float* r);
#define MWC_HLEVEL(BIT, C0, C1, M0, M1)                                                                    \
    template <> __device__ __forceinline__ void dpp_hi_level<BIT, 1>(const float* x, float* r) {          \
        asm("s_nop 1\n\t" MWC_HADD(0, 1, 2, C0, C1, M0, M1) : "=&v"(r[0]) : "v"(x[0]), "v"(x[1]));         \
    }                                                                                                      \
    template <> __device__ __forceinline__ void dpp_hi_level<BIT, 2>(const float* x, float* r) {          \
        asm("s_nop 1\n\t" MWC_HADD(0, 2, 3, C0, C1, M0, M1) MWC_HADD(1, 4, 5, C0, C1, M0, M1)              \
            : "=&v"(r[0]), "=&v"(r[1])                                                                     \
            : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]));                                                 \
    }                                                                                                      \
    template <> __device__ __forceinline__ void dpp_hi_level<BIT, 4>(const float* x, float* r) {          \
        asm("s_nop 1\n\t" MWC_HADD(0, 4, 5, C0, C1, M0, M1) MWC_HADD(1, 6, 7, C0, C1, M0, M1)              \
                MWC_HADD(2, 8, 9, C0, C1, M0, M1) MWC_HADD(3, 10, 11, C0, C1, M0, M1)                      \
            : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])                                           \
            : "v"(x[0]), "v"(x[1]), "v"(x[2]), "v"(x[3]), "v"(x[4]), "v"(x[5]), "v"(x[6]), "v"(x[7]));     \
    }                                                                                                      \
    template <> __device__ __forceinline__ void dpp_hi_level<BIT, 8>(const float* x, float* r) {          \
        dpp_hi_level<BIT, 4>(x, r);                                                                        \
        dpp_hi_level<BIT, 4>(x + 8, r + 4);                                                                \
    }
MWC_HLEVEL(3, "row_ror:8", "row_ror:8", "0x3", "0xc")
MWC_HLEVEL(2, "row_shl:4", "row_shr:4", "0x5", "0xa")
#undef MWC_HLEVEL
#undef MWC_HADD

// x + its partner's x at a single-value level
template <int BIT> __device__ __forceinline__ float hi_single(float x) {
    float r;
    if constexpr (BIT == 3) {
        asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %1 row_ror:8 row_mask:0xf bank_mask:0xf" : "=v"(r) : "v"(x));
    } else if constexpr (BIT == 2) {
        asm("s_nop 1\n\t"
            "v_add_f32_dpp %0, %1, %1 row_shl:4 row_mask:0xf bank_mask:0x5\n\t"
            "v_add_f32_dpp %0, %1, %1 row_shr:4 row_mask:0xf bank_mask:0xa"
            : "=&v"(r)
            : "v"(x));
    } else {
        float pair[2] = {x, x};
        permlane_swap_pairs<BIT, 1>(pair);
        r = pair[0] + pair[1];
    }
    return r;
}

// One reduce-scatter level on lane bit PB for NP value pairs (x[2q], x[2q+1]): lanes whose bit PB is 0
// get x[2q] + the partner's x[2q], the others x[2q+1] + the partner's x[2q+1] (partner = lane ^ 2^PB).
// Bits 2 and 3 are bank-masked DPP reads, 4 and 5 permlane swaps, 0 and 1 selects and a DPP add.
template <int PB, int NP> __device__ __forceinline__ void pair_level(const float* x, float* r, int lane) {
    if constexpr (PB == 2 || PB == 3) {
        dpp_hi_level<PB, NP>(x, r);
    } else if constexpr (PB == 4 || PB == 5) {
        float t[2 * NP];
#pragma unroll
        for (int q = 0; q < 2 * NP; ++q) t[q] = x[q];
        permlane_swap_pairs<PB, NP>(t);
#pragma unroll
        for (int q = 0; q < NP; ++q) r[q] = t[2 * q] + t[2 * q + 1];
    } else {
        const bool hi = ((lane >> PB) & 1) != 0;
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            const float keep = hi ? x[2 * q + 1] : x[2 * q];
            const float send = hi ? x[2 * q] : x[2 * q + 1];
            r[q] = keep + dpp_flip<PB>(send);
        }
    }
}

template <int CPW, int V, int L = 0, int M = V>
__device__ __forceinline__ float reduce_scatter_hi_lv(float (&x)[V]) {
    constexpr int B = hi_bit<CPW>(L);
    static_assert(B != 0 && B != 1, "lane bits 0 and 1 are not part of a channel's lane group here");
    if constexpr (B < 0) {
        return x[0];
    } else if constexpr (M > 1) {
        if constexpr (B >= 4) {
            permlane_swap_pairs<B, M / 2>(x);
#pragma unroll
            for (int q = 0; q < M / 2; ++q) x[q] = x[2 * q] + x[2 * q + 1];
        } else {
            float r[M / 2];
            dpp_hi_level<B, M / 2>(x, r);
#pragma unroll
            for (int q = 0; q < M / 2; ++q) x[q] = r[q];
        }
        return reduce_scatter_hi_lv<CPW, V, L + 1, M / 2>(x);
    } else {
        x[0] = hi_single<B>(x[0]);
        return reduce_scatter_hi_lv<CPW, V, L + 1, 1>(x);
    }
}
// x is clobbered; V (a power of two) values, 2 <= V <= 64/CPW.
template <int CPW, int V> __device__ __forceinline__ float reduce_scatter_hi(float (&x)[V]) {
    static_assert(V >= 2 && (V & (V - 1)) == 0 && V * CPW <= 64, "shape");
    return reduce_scatter_hi_lv<CPW, V>(x);
}

}  // namespace mwc

#define MWC_HIP_TRY(expr)                                  \
    do {                                                   \
        hipError_t _e = (expr);                            \
        if (_e != hipSuccess) return mwc_set_hip_error(_e, #expr); \
    } while (0)

int mwc_set_error(int status, const char* msg);
int mwc_set_hip_error(hipError_t e, const char* what);
