// Shared device/host helpers for the gfx950 kernels of the MI355X execution provider.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <type_traits>

#include "../../include/ortmi_kernels.h"

namespace ortmi {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

// Largest split-partial array a one-token attention hands to the o_proj GEMV
// (fp32 floats, all heads): the GEMV's workgroups stage it in LDS (32 KB).
constexpr int kDecodeMergeMaxFloats = 8192;

// Buffer resource word 3 for raw (untyped) buffer loads and stores on gfx9-family
// GPUs. A raw buffer access whose offset is at or past the resource's byte count
// touches no memory: a load returns zeros and a store is dropped.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of a buffer load or store that marks it non-temporal.
constexpr int kCachePolicyNT = 2;

template <typename P>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const P* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<P*>(base), 0, (int)bytes, kBufferWord3);
}

// MI355X dispatches the workgroups of a 1-D grid round-robin over its 8 XCDs
// (each with its own L2): workgroup i runs on XCD i % 8 as that XCD's (i / 8)-th.
constexpr int kXcds = 8;

// ---------------------------------------------------------------- dtype IO --
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(half_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(uint16_t bf) {  // bfloat16 bits
    return __uint_as_float((uint32_t)bf << 16);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ half_t from_f32<half_t>(float x) { return (half_t)x; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float x) {  // bf16, RNE
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Round a float to the storage dtype and widen it back (models a tensor that the
// reference materialises in the op dtype).
template <typename T>
__device__ __forceinline__ float round_to(float x) { return to_f32(from_f32<T>(x)); }

// ------------------------------------------------------------ reductions --
// Cross-lane reductions without the LDS permute path: inside a 16-lane row the
// partner values come from DPP moves (quad_perm [1,0,3,2], quad_perm [2,3,0,1],
// row_half_mirror, row_mirror), which after the two quad steps pair every lane
// with a lane holding the other part of its group; across rows the gfx950
// v_permlane16_swap / v_permlane32_swap exchange the halves of 32 / 64 lanes.
// Every lane of a group ends with the same value (the combining operations are
// commutative). All lanes of the wave must be active. The moves are written with
// a zero "old" value, full row/bank masks and bound_ctrl, which lets the compiler
// fold each one into its consumer (v_add_f32_dpp, v_max_f32_dpp): one instruction
// per step. Every pattern used here reads a lane inside the same row.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
struct LanePair {
    float a, b;
};
__device__ __forceinline__ LanePair swap16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, v),
                                                    __builtin_bit_cast(unsigned, v), false, false);
    return {__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1])};
}
__device__ __forceinline__ LanePair swap32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, v),
                                                    __builtin_bit_cast(unsigned, v), false, false);
    return {__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1])};
}

// Sum over aligned groups of `W` lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (W >= 2) v += dpp_mov<0xB1>(v);
    if constexpr (W >= 4) v += dpp_mov<0x4E>(v);
    if constexpr (W >= 8) v += dpp_mov<0x141>(v);
    if constexpr (W >= 16) v += dpp_mov<0x140>(v);
    if constexpr (W >= 32) {
        const LanePair p = swap16(v);
        v = p.a + p.b;
    }
    if constexpr (W >= 64) {
        const LanePair p = swap32(v);
        v = p.a + p.b;
    }
    return v;
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (W >= 2) v = fmaxf(v, dpp_mov<0xB1>(v));
    if constexpr (W >= 4) v = fmaxf(v, dpp_mov<0x4E>(v));
    if constexpr (W >= 8) v = fmaxf(v, dpp_mov<0x141>(v));
    if constexpr (W >= 16) v = fmaxf(v, dpp_mov<0x140>(v));
    if constexpr (W >= 32) {
        const LanePair p = swap16(v);
        v = fmaxf(p.a, p.b);
    }
    if constexpr (W >= 64) {
        const LanePair p = swap32(v);
        v = fmaxf(p.a, p.b);
    }
    return v;
}
// Sum over the lanes that share (lane % LPR), i.e. across the 64 / LPR aligned
// groups of LPR lanes (LPR in {8, 16, 32}).
template <int LPR>
__device__ __forceinline__ float across_groups_sum(float v) {
    static_assert(LPR == 8 || LPR == 16 || LPR == 32, "group width");
    if constexpr (LPR == 8) v += dpp_mov<0x128>(v);  // row_ror:8 = lane ^ 8 in a row
    if constexpr (LPR <= 16) {
        const LanePair p = swap16(v);
        v = p.a + p.b;
    }
    const LanePair p = swap32(v);
    return p.a + p.b;
}
__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }
__device__ __forceinline__ float wave_max(float v) { return group_max<64>(v); }

__device__ __forceinline__ int nibble(uint8_t byte, int hi) { return hi ? (byte >> 4) : (byte & 0x0f); }

// ------------------------------------------------ int4 x fp16 dot products --
// Reorder 8 activations [a0..a7] to the pair order [a0,a4,a1,a5,a2,a6,a3,a7] used by
// the dequantised weights (an identical permutation of k on both MFMA operands).
__device__ __forceinline__ uint4 permute_act8(uint4 v) {
    return make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u),
                      __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                      __builtin_amdgcn_perm(v.w, v.y, 0x05040100u),
                      __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
}

// fp16 activations as pairs: sum over the 32 codes of one chunk of a * (q - zp).
// `av` holds the chunk's activations in pair order (a_j, a_j+4) for each 8-code
// word, the order dequant_word_pairs gives the codes in; (1024 + q) - (1024 + zp)
// is exact in fp16, v_dot2_f32_f16 multiplies exactly and accumulates in fp32.
__device__ __forceinline__ float dot32_pairs(const uint4 (&av)[4], uint4 w, half2_t zoff) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t aw[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t m = ((words[i] >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
            const half2_t q = __builtin_bit_cast(half2_t, m) - zoff;
            const half2_t a = __builtin_bit_cast(half2_t, aw[j]);
            if (j & 1) d1 = __builtin_amdgcn_fdot2(a, q, d1, false);
            else d0 = __builtin_amdgcn_fdot2(a, q, d0, false);
        }
    }
    return d0 + d1;
}



// --------------------------------------------------------------- host side --
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);
int device_cu_count();

#define ORTMI_REQUIRE(cond, msg)                                 \
    do {                                                         \
        if (!(cond)) return ::ortmi::fail(ORTMI_E_INVALID, msg); \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace ortmi
