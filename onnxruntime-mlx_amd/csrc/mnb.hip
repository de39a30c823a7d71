// MatMulNBits (com.microsoft) for gfx950.
//
// ORT layout, read in place (no repack): B is [N, nb, bs*bits/8] uint8 with
// blocks consecutive along K, so row n is nb*bs*bits/8 contiguous bytes and each
// byte holds k (low nibble) and k+1 (high nibble). Scales are [N, nb] in the
// activation dtype; 4-bit zero points are packed [N, ceil(nb/2)], low nibble for
// even blocks.
//
// Kernels:
//  * mnb_gemv4  - decode (M == 1), bits 4, bs in {32, 64, 128}. HBM-bound: each
//    lane owns a contiguous run of 32-code chunks of K and keeps the matching
//    activations in VGPRs (staged once per workgroup through LDS), then streams
//    rows of B with 128-bit range-checked buffer loads, a ring of row groups in
//    flight per wave. fp32/bf16 activations: zero points folded as
//    s*(sum(a*q) - zp*sum(a)), one byte-convert and one FMA per code. fp16
//    activations: codes become exact fp16 (q - zp) pairs and v_dot2_f32_f16
//    takes two codes per instruction.
//  * mnb_gemm4  - prefill (M > 1, fp16 or bf16), bits 4, bs in {32, 64, 128}.
//    MFMA v_mfma_f32_32x32x16_f16 / _bf16: the weight tile is dequantised to the
//    activation dtype (fp16((q - zp) * s) or bf16((q - zp) * s), one rounding)
//    and the activation tile is staged in LDS; fp32 accumulation, one rounding of Y.
//  * mnb_generic - every other form (bits 8, bs 16, fp32 prefill): fp32 dequant
//    to LDS and a VALU tile product.
#include "common.h"

namespace ortmi {

// -------------------------------------------------------------- GEMV (M=1) --

// Dot product of 32 activations with the 32 4-bit codes of one 16-byte chunk.
// Code i of the chunk is nibble (i & 1) of byte i/2, i.e. bits [4i, 4i+4) of the
// little-endian 128-bit word.
//
// The codes are converted two at a time by the fp8 (e4m3) pack convert: a byte
// 0000qqqq read as e4m3 is q * 2^-9 exactly (a subnormal m * 2^-9 for q < 8,
// (8 + m) * 2^-9 with exponent field 1 for q >= 8), so the sum comes out scaled
// by the exact power of two code_unit() and the caller scales it back. Scaling
// by a power of two commutes with every rounding here, so the result equals the
// unscaled sum bit for bit. One instruction per two codes, against a bit-field
// extract plus a byte convert per code.
__device__ __forceinline__ float dot32_codes(const float* a, uint4 w) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = words[i] & 0x0F0F0F0Fu;         // codes 8i+0,2,4,6
        const uint32_t hi = (words[i] >> 4) & 0x0F0F0F0Fu;  // codes 8i+1,3,5,7
        const float* ai = a + 8 * i;
        const auto l01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, false);
        const auto l23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)lo, true);
        const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
        const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
        d0 = fmaf(ai[0], l01[0], d0);
        d1 = fmaf(ai[1], h01[0], d1);
        d0 = fmaf(ai[2], l01[1], d0);
        d1 = fmaf(ai[3], h01[1], d1);
        d0 = fmaf(ai[4], l23[0], d0);
        d1 = fmaf(ai[5], h23[0], d1);
        d0 = fmaf(ai[6], l23[1], d0);
        d1 = fmaf(ai[7], h23[1], d1);
    }
    return d0 + d1;
}
// The value dot32_codes gives code 1 (2^-9 for e4m3), read from the hardware.
__device__ __forceinline__ float code_unit() {
    return __builtin_amdgcn_cvt_pk_f32_fp8(1, false)[0];
}

// Activations live in LDS as fp32 in 16-byte units. Lane l reads the 8*CPL
// consecutive units of its chunks; unit u of lane l is stored at
// u ^ ((u / (8*CPL)) & 7), so the 8 lanes of one read phase hit 8 bank groups.
template <int CPL>
__device__ __forceinline__ int act_unit(int u) {
    return u ^ ((u / (8 * CPL)) & 7);
}

// Zero-point bytes that cover the blocks of one lane's CPL chunks, worst case
// over the 64 lanes (4-bit zero points: two blocks per byte).
constexpr int zp_window(int BS, int CPL) {
    int most = 1;
    for (int l = 0; l < 64; ++l) {
        const int c0 = l * CPL;
        const int b0 = (32 * c0) / BS / 2, b1 = (32 * (c0 + CPL - 1)) / BS / 2;
        if (b1 - b0 + 1 > most) most = b1 - b0 + 1;
    }
    return most;
}

// One group of R rows as loaded: weights, scales and zero-point bytes are kept
// raw and converted only when the group is reduced, so no instruction consumes a
// prefetched value before its row is needed (a conversion at load time would
// make the compiler wait for the prefetch there).
template <typename T, int R, int CPL, int ZB>
struct GemvGroup {
    uint4 w[R][CPL];
    T s[R][CPL];
    uint8_t z[R][ZB];
};

// Lane l owns the CPL consecutive 32-code chunks [l*CPL, (l+1)*CPL) of every row,
// so a row costs one 16*CPL-byte weight run, CPL adjacent scales and one or two
// zero-point bytes per lane; or (IL, fp16 rows of whole 64-chunk runs at block 32)
// chunks l, l + 64, ..., so each of the row's CPL weight loads reads 1 KB
// contiguous, each scale load 128 bytes, with one zero-point byte per chunk. The
// activation loads are issued first, then the weight loads of the wave's first D
// row groups; the activations go through LDS
// (one copy per workgroup) into VGPRs while the weights are in flight. Row groups
// of R rows are dealt to waves round-robin; a ring of D groups keeps the next
// D - 1 groups' loads in flight while one group is reduced.
// Activations in VGPRs: fp32 (32 per chunk) for fp32/bf16, fp16 pairs (16 VGPRs
// per chunk, v_dot2 products) for fp16 (H2).
// Optional fusions of the decoder's neighbours into the GEMV (decode only):
//  * prologue: the activation row is (Skip)SimplifiedLayerNorm(x [+ skip]) * gamma,
//    computed by every workgroup from x (K elements) before staging; workgroup 0
//    also writes the residual x + skip. Rounding as the unfused ops: the sum is
//    rounded to T, the normalised value once more.
//  * SwiGLU pairs: rows come interleaved (gate row i, up row i), a wave takes both
//    rows of a pair and writes Y[i] = (g * sigmoid(g)) * u, each op rounded to T as
//    the Sigmoid/Mul/Mul graph stores it.
//  * split merge (MRG): the activation row is attention output still held as
//    split partials [heads][splits][hd + 2] (o, max, sum) by the one-token decode;
//    each workgroup merges them as the merge kernel would, rounding to T.
template <typename T>
struct GemvPrologue {
    const T* skip;
    const T* gamma;
    T* residual;
    float eps;
    const float* part = nullptr;
    int splits = 0;
    int hd = 0;
};

// One scale, or an aligned pair of scales, through a buffer load.
template <typename T>
__device__ __forceinline__ T load_scale(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
    } else {
        return __builtin_bit_cast(T, (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
    }
}
template <typename T>
__device__ __forceinline__ void load_scale_pair(__amdgpu_buffer_rsrc_t r, uint32_t off, T& a, T& b) {
    if constexpr (sizeof(T) == 4) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        a = __builtin_bit_cast(T, (uint32_t)v[0]);
        b = __builtin_bit_cast(T, (uint32_t)v[1]);
    } else {
        const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
        a = __builtin_bit_cast(T, (uint16_t)(v & 0xffffu));
        b = __builtin_bit_cast(T, (uint16_t)(v >> 16));
    }
}

// Split-merge prologue bounds: partial floats per workgroup (one batch of
// float4 loads, kMergeVec per thread).
constexpr int kMergeVec = kDecodeMergeMaxFloats / (256 * 4);

// LDS bytes of the staged activation row (fp16 pairs or fp32 units).
template <typename T, bool H2>
constexpr size_t gemv_stage_bytes(int Kp) {
    return (size_t)Kp * (H2 ? sizeof(half_t) : sizeof(float));
}
// LDS bytes of the split-merge prologue: partials, split weights, 1/L per head.
static inline size_t gemv_merge_bytes(int K, int hd, int splits) {
    const size_t nh = (size_t)K / hd, nparts = nh * splits * (hd + 2);
    return (((nparts + 3) & ~(size_t)3) + nh * splits + nh) * sizeof(float);
}

template <typename T, int BS, int CPL, int R, int D, bool PRO = false, bool PAIR = false,
          bool SV = false, bool H2 = std::is_same<T, half_t>::value, bool NT = true,
          bool MRG = false, int RW = 1, bool IL = false>
__global__ __launch_bounds__(256) void mnb_gemv4_kernel(const T* __restrict__ A,
                                                        const uint8_t* __restrict__ B,
                                                        const T* __restrict__ S,
                                                        const uint8_t* __restrict__ Z,
                                                        T* __restrict__ Y, int N, int K,
                                                        int nb, GemvPrologue<T> pro) {
    static_assert(!PAIR || R == 2, "SwiGLU pairs take two rows per group");
    static_assert(!H2 || std::is_same<T, half_t>::value, "fp16 pairs need fp16 activations");
    static_assert(D >= 1, "ring depth");
    static_assert(!IL || (H2 && !SV && BS == 32), "interleaved chunks: fp16 pairs, block 32");
    extern __shared__ float4 sA[];
    __shared__ float s_red[4];
    constexpr int ZB = IL ? CPL : zp_window(BS, CPL);
    using Group = GemvGroup<T, R, CPL, ZB>;
    const int Kp = nb * BS;
    const int C = Kp / 32;  // 32-code chunks per row
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves_total = gridDim.x * 4;
    // A wave works on RW units of R rows at once, LR = 64 / RW lanes per unit
    // (RW > 1 when a row has few chunks, so that no lane idles); a group is RW
    // consecutive units.
    constexpr int LR = 64 / RW;
    const int li = lane % LR, slot = lane / LR;
    const int nunits = (N + R - 1) / R;
    const int ngroups = (nunits + RW - 1) / RW;
    const size_t row_bytes = (size_t)Kp / 2;
    const int zp_cols = (nb + 1) / 2;
    const int c0 = li * CPL;
    // Chunk j of this lane: CPL consecutive chunks, or (IL) chunks li + j * LR, so
    // that each load instruction of a unit reads one contiguous run.
    auto chunk = [&](int j) { return IL ? li + j * LR : c0 + j; };

    // 1. activation loads (16 bytes each), all in flight before anything else.
    constexpr int EPL = 16 / sizeof(T);
    // Kp <= 64 lanes * CPL * 32 codes, so 256 threads need ceil(8 * CPL / EPL) vectors each.
    constexpr int AV = (8 * CPL + EPL - 1) / EPL;
    const int nvec = Kp / EPL;
    const bool vec_ok = (K % EPL) == 0 && (reinterpret_cast<uintptr_t>(A) % 16) == 0;
    uint4 av[AV];
    auto load_vec = [&](const T* src, int u) -> uint4 {
        const int vi = threadIdx.x + u * 256;
        const int k0 = vi * EPL;
        if (vi < nvec && vec_ok && k0 + EPL <= K) return *reinterpret_cast<const uint4*>(src + k0);
        T t[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e)
            t[e] = (vi < nvec && k0 + e < K) ? src[k0 + e] : from_f32<T>(0.f);
        return *reinterpret_cast<const uint4*>(t);
    };
    // Split merge: the whole partial array in one batch of loads (at most
    // kMergeVec float4 per thread; the launcher checks the size).
    float4 pbuf[MRG ? kMergeVec : 1];
    float ptail = 0.f;
    if constexpr (MRG) {
        const int nparts = (K / pro.hd) * pro.splits * (pro.hd + 2);
#pragma unroll
        for (int u = 0; u < kMergeVec; ++u) {
            const int idx = threadIdx.x + 256 * u;
            pbuf[u] = idx < nparts / 4 ? reinterpret_cast<const float4*>(pro.part)[idx]
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (threadIdx.x < (nparts & 3)) ptail = pro.part[(nparts & ~3) + threadIdx.x];
    } else {
#pragma unroll
        for (int u = 0; u < AV; ++u) av[u] = load_vec(A, u);
    }
    uint4 skv[PRO ? AV : 1], gmv[PRO ? AV : 1];
    if constexpr (PRO) {
#pragma unroll
        for (int u = 0; u < AV; ++u) {
            skv[u] = pro.skip ? load_vec(pro.skip, u) : make_uint4(0, 0, 0, 0);
            gmv[u] = load_vec(pro.gamma, u);
        }
    }

    // 2. weights of the first D row groups, issued after the activation loads (a
    // wait on a load also waits on every load issued before it). Loads never
    // branch, which keeps every wait on a prefetch exact: they are buffer loads,
    // and a group past the end, or a chunk past the row end, gets an offset past
    // the buffer's range, which returns zeros without a memory access (a zero chunk
    // meets zero activations, a missing group is never reduced). The last group's
    // second row, when N is odd, repeats row N - 1 (in bounds).
    const int g0 = blockIdx.x * 4 + wave;
    const int blk0 = (32 * min(c0, C - 1)) / BS;
    const uint32_t b_end = (uint32_t)((size_t)N * row_bytes);
    const uint32_t s_end = (uint32_t)((size_t)N * nb * sizeof(T));
    const uint32_t z_end = (uint32_t)((size_t)N * zp_cols);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B), 0, (int)b_end, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(S), 0, (int)s_end, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(Z ? Z : B), 0, Z ? (int)z_end : 0, kBufferWord3);
    // A unit past the end in a live group repeats the last unit (in bounds; its
    // lanes then store the same values to the same rows).
    auto unit_of = [&](int gi) { return min(gi * RW + slot, nunits - 1); };
    auto load_group = [&](Group& g, int gi) {
        const bool live = gi < ngroups;
        const int unit = unit_of(gi);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = min(unit * R + r, N - 1);
            const uint32_t zoff = live ? (uint32_t)(n * zp_cols) : z_end;
#pragma unroll
            for (int t = 0; t < ZB; ++t) {
                // Loaded either way (no records without Z): no load behind a branch.
                const int zcol = IL ? min(chunk(t), C - 1) / 2 : blk0 / 2 + t;
                const uint8_t zb = (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(
                    rz, zoff + (uint32_t)min(zcol, zp_cols - 1), 0, 0);
                g.z[r][t] = Z ? zb : (uint8_t)0x88;
            }
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int c = chunk(j);
                const bool ok = live && c < C;
                const uint32_t boff = ok ? (uint32_t)((size_t)n * row_bytes) + 16u * c : b_end;
                // Streamed once: optionally non-temporal (cache policy nt).
                const u32x4_t v =
                    __builtin_amdgcn_raw_buffer_load_b128(rb, boff, 0, NT ? kCachePolicyNT : 0);
                g.w[r][j] = make_uint4(v.x, v.y, v.z, v.w);
                if constexpr (!SV) {
                    const uint32_t soff =
                        ok ? (uint32_t)(((size_t)n * nb + (32 * c) / BS) * sizeof(T)) : s_end;
                    g.s[r][j] = load_scale<T>(rs, soff);
                }
            }
            if constexpr (SV) {
                // Block 32 and an even CPL: the lane's scales are CPL/2 aligned pairs.
#pragma unroll
                for (int j = 0; j < CPL; j += 2) {
                    const int c = c0 + j;
                    const uint32_t soff =
                        live && c < C ? (uint32_t)(((size_t)n * nb + c) * sizeof(T)) : s_end;
                    load_scale_pair(rs, soff, g.s[r][j], g.s[r][j + 1]);
                }
            }
        }
    };
    Group g[D];
#pragma unroll
    for (int d = 0; d < D; ++d) load_group(g[d], g0 + d * waves_total);

    if constexpr (MRG) {
        // Partials -> LDS (after the staging area), then per head h the split
        // weights e^(m_i - M) and 1 / sum_i w_i l_i, then activation k = h*hd + d
        // as (sum_i w_i o_i[d]) / L, rounded to T as the merge kernel stores it.
        const int nh = K / pro.hd, ns = pro.splits, stride = pro.hd + 2;
        const int nparts = nh * ns * stride;
        float* sP = reinterpret_cast<float*>(reinterpret_cast<char*>(sA) + gemv_stage_bytes<T, H2>(Kp));
        float* sW = sP + ((nparts + 3) & ~3);
        float* sInv = sW + nh * ns;
#pragma unroll
        for (int u = 0; u < kMergeVec; ++u) {
            const int idx = threadIdx.x + 256 * u;
            if (idx < nparts / 4) reinterpret_cast<float4*>(sP)[idx] = pbuf[u];
        }
        if (threadIdx.x < (nparts & 3)) sP[(nparts & ~3) + threadIdx.x] = ptail;
        __syncthreads();
        for (int h = threadIdx.x; h < nh; h += 256) {
            const float* ph = sP + h * ns * stride;
            float M = -INFINITY;
            for (int i = 0; i < ns; ++i) M = fmaxf(M, ph[i * stride + pro.hd]);
            float L = 0.f;
            for (int i = 0; i < ns; ++i) {
                const float mi = ph[i * stride + pro.hd];
                const float w = mi == -INFINITY ? 0.f : __expf(mi - M);
                sW[h * ns + i] = w;
                L += w * ph[i * stride + pro.hd + 1];
            }
            sInv[h] = L > 0.f ? 1.0f / L : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < AV; ++u) {
            const int vi = threadIdx.x + u * 256;
            const int k0 = vi * EPL;
            T t[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) t[e] = from_f32<T>(0.f);
            if (vi < nvec && k0 < K) {
                const int h = k0 / pro.hd, d0 = k0 % pro.hd;
                const float* ph = sP + h * ns * stride + d0;
                const float* wh = sW + h * ns;
                float acc[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
                for (int i = 0; i < ns; ++i) {
                    const float w = wh[i];
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[e] = fmaf(ph[i * stride + e], w, acc[e]);
                }
#pragma unroll
                for (int e = 0; e < EPL; ++e) t[e] = from_f32<T>(acc[e] * sInv[h]);
            }
            av[u] = *reinterpret_cast<const uint4*>(t);
        }
    }

    // 3. activations (normalised first when fused) -> LDS -> VGPRs.
    float scale_all = 1.f;
    if constexpr (PRO) {
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < AV; ++u) {
            const int vi = threadIdx.x + u * 256;
            if (vi >= nvec) continue;
            T* t = reinterpret_cast<T*>(&av[u]);
            const T* k = reinterpret_cast<const T*>(&skv[u]);
#pragma unroll
            for (int e = 0; e < EPL; ++e) {
                float v = to_f32(t[e]);
                if (pro.skip) v = round_to<T>(v + to_f32(k[e]));
                t[e] = from_f32<T>(v);
                ss += v * v;
            }
            if (pro.residual && blockIdx.x == 0) {
                const int k0 = vi * EPL;
                if (vec_ok && k0 + EPL <= K) {
                    *reinterpret_cast<uint4*>(pro.residual + k0) = av[u];
                } else {
                    for (int e = 0; e < EPL; ++e)
                        if (k0 + e < K) pro.residual[k0 + e] = t[e];
                }
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) s_red[wave] = ss;
        __syncthreads();
        scale_all = 1.0f / sqrtf((s_red[0] + s_red[1] + s_red[2] + s_red[3]) / (float)K + pro.eps);
    }
#pragma unroll
    for (int u = 0; u < AV; ++u) {
        const int vi = threadIdx.x + u * 256;
        if (vi >= nvec) continue;
        T* t = reinterpret_cast<T*>(&av[u]);
        if constexpr (H2) {
            // 8 halfs = one 8-code word: one 16-byte unit in pair order.
            if constexpr (PRO) {
                const T* gm = reinterpret_cast<const T*>(&gmv[u]);
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    t[e] = from_f32<T>(to_f32(t[e]) * scale_all * to_f32(gm[e]));
            }
            reinterpret_cast<uint4*>(sA)[vi] = permute_act8(av[u]);
        } else {
            float f[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) f[e] = to_f32(t[e]);
            if constexpr (PRO) {
                const T* gm = reinterpret_cast<const T*>(&gmv[u]);
#pragma unroll
                for (int e = 0; e < EPL; ++e) f[e] = round_to<T>(f[e] * scale_all * to_f32(gm[e]));
            }
#pragma unroll
            for (int e = 0; e < EPL; e += 4) {
                const int q = (vi * EPL + e) / 4;
                sA[act_unit<CPL>(q)] = make_float4(f[e], f[e + 1], f[e + 2], f[e + 3]);
            }
        }
    }
    __syncthreads();
    // fp32 form: a[j][*] and asum[j]; fp16 pairs: ah[j][*] (the other form is unused).
    float a[H2 ? 1 : CPL][32];
    float asum[H2 ? 1 : CPL];
    uint4 ah[H2 ? CPL : 1][4];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = chunk(j);
        if constexpr (H2) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                ah[j][i] = c < C ? reinterpret_cast<const uint4*>(sA)[4 * c + i]
                                 : make_uint4(0, 0, 0, 0);
        } else {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 v =
                    c < C ? sA[act_unit<CPL>(8 * c + i)] : make_float4(0.f, 0.f, 0.f, 0.f);
                a[j][4 * i + 0] = v.x;
                a[j][4 * i + 1] = v.y;
                a[j][4 * i + 2] = v.z;
                a[j][4 * i + 3] = v.w;
                s += (v.x + v.y) + (v.z + v.w);
            }
            asum[j] = s * code_unit();  // in dot32_codes' scaled units (exact)
        }
    }
    // Back from dot32_codes' units: an exact power of two.
    const float code_scale = H2 ? 1.f : 1.0f / code_unit();

    auto reduce_store = [&](const Group& gr, int gi) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float total = 0.f;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const int blk = (32 * min(chunk(j), C - 1)) / BS;
                const int d = blk / 2 - blk0 / 2;
                uint8_t zbyte = gr.z[r][0];
                if constexpr (IL) {
                    zbyte = gr.z[r][j];
                } else {
#pragma unroll
                    for (int t = 1; t < ZB; ++t)
                        if (d == t) zbyte = gr.z[r][t];
                }
                const int zq = nibble(zbyte, blk & 1);
                if constexpr (H2) {
                    const half_t zo = (half_t)(1024 + zq);
                    const half2_t zoff = {zo, zo};
                    total = fmaf(to_f32(gr.s[r][j]), dot32_pairs(ah[j], gr.w[r][j], zoff), total);
                } else {
                    const float d32 = dot32_codes(a[j], gr.w[r][j]);
                    total = fmaf(to_f32(gr.s[r][j]), d32 - (float)zq * asum[j], total);
                }
            }
            acc[r] = total * code_scale;
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = group_sum<LR>(acc[r]);
        // Every lane of a unit holds its sums and every lane stores (same-address
        // writes of a wave coalesce).
        const int unit = unit_of(gi);
        if constexpr (PAIR) {
            const float gv = round_to<T>(acc[0]), up = round_to<T>(acc[1]);
            const float sig = round_to<T>(1.0f / (1.0f + __expf(-gv)));
            Y[unit] = from_f32<T>(round_to<T>(gv * sig) * up);
            return;
        }
        const int r = li % R;
        float v = acc[0];
#pragma unroll
        for (int i = 1; i < R; ++i)
            if (r == i) v = acc[i];
        Y[min(unit * R + r, N - 1)] = from_f32<T>(v);
    };

    for (int gi = g0; gi < ngroups; gi += D * waves_total) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int idx = gi + d * waves_total;
            if (idx >= ngroups) return;
            reduce_store(g[d], idx);
            load_group(g[d], idx + D * waves_total);
        }
    }
}

// Launch of one kernel instance: `grid` workgroups of 4 waves.
template <typename T, int BS, int CPL, int R, int D, bool PRO, bool PAIR, bool SV, bool H2,
          bool NT = true, bool MRG = false, int RW = 1, bool IL = false>
static int launch_gemv4_inst(const T* A, const uint8_t* B, const T* S, const uint8_t* Z, T* Y,
                             int N, int K, int nb, const GemvPrologue<T>& pro, long grid,
                             hipStream_t st) {
    size_t lds = gemv_stage_bytes<T, H2>(nb * BS);
    if constexpr (MRG) lds += gemv_merge_bytes(K, pro.hd, pro.splits);
    hipLaunchKernelGGL((mnb_gemv4_kernel<T, BS, CPL, R, D, PRO, PAIR, SV, H2, NT, MRG, RW, IL>),
                       dim3((unsigned)grid), dim3(256), lds, st, A, B, S, Z, Y, N, K, nb, pro);
    return check_launch("mnb_gemv4");
}

// Grid, ring depth and cache policy per shape, from sweeps on MI355X with the
// weights streamed from HBM (the decoder's N x K = 2048 x 1536, 1536 x 1536,
// 17920 x 1536 in pairs, 1536 x 8960 and 151936 x 1536 in fp16, and 11008 x 4096
// in fp32). Groups per wave: 1 while the groups fit about 10 waves per CU, 2 for
// K > 4096 fp16 (activations fill the VGPRs), about 3.6 (3 workgroups per CU) for
// K = 4096, 3 up to about 80 groups per CU, 16 beyond. A ring of 2, of 1 when
// the activations fill the VGPRs, of 4 for the long walks. Weights non-temporal
// except for those two cases, which measured faster with cached loads.
template <typename T, int BS, int CPL, bool PRO, bool PAIR, bool MRG>
static int launch_gemv4_cpl(const T* A, const uint8_t* B, const T* S, const uint8_t* Z, T* Y,
                            int N, int K, int nb, const GemvPrologue<T>& pro, hipStream_t st) {
    constexpr int R = PAIR ? 2 : 1;
    constexpr bool H2 = std::is_same<T, half_t>::value;
    const long groups = ((long)N + R - 1) / R;
    const long cus = device_cu_count();
    const bool longwalk = groups > 80 * cus;
    long grid;
    if (longwalk) grid = (groups + 63) / 64;
    else if (CPL >= 3) grid = (groups + 7) / 8;
    // With the split-merge prologue every workgroup merges the whole activation
    // row first: fewer, fuller workgroups (o_proj 1536x1536: 384 -> 256
    // workgroups, 5.13 -> 4.87 us).
    else if (MRG && groups <= 10 * cus) grid = (groups + 5) / 6;
    else if (groups <= 10 * cus) grid = (groups + 3) / 4;
    // Three workgroups per CU: K = 4096, N = 11008 measured 8.1 us against 8.6 us at
    // four (fp32 and fp16 alike); grids that are not a multiple of the CU count
    // (2.5 or 3.5 per CU) measured slowest.
    else if (CPL >= 2) grid = std::min((groups + 3) / 4, 3 * cus);
    else grid = (groups + 11) / 12;
    bool sv = false;
    if constexpr (BS == 32 && CPL % 2 == 0)  // scale pairs as one load when every lane's pair is aligned
        sv = nb % 2 == 0 && (reinterpret_cast<uintptr_t>(S) % (2 * sizeof(T))) == 0 && nb >= 2;
    constexpr bool kSV = BS == 32 && CPL % 2 == 0;
#define ORTMI_GEMV_INST(DV, SVV, NTV)                                                              \
    return launch_gemv4_inst<T, BS, CPL, R, DV, PRO, PAIR, SVV, H2, NTV, MRG>(A, B, S, Z, Y, N, K, \
                                                                             nb, pro, grid, st)
    // Interleaved chunks (lane l owns chunks l, l + 64, ...: every weight load of a
    // row one contiguous 1 KB run) for fp16 rows of a whole number of 64-chunk runs,
    // with non-temporal loads. Measured on MI355X in graph replay against the
    // consecutive chunks: 4096 x 14336 13.4 -> 11.8 us, 3072 x 8192 9.1 -> 6.8 us,
    // 8192 x 8192 (zero points) 14.8 -> 13.3 us, 4096 x 4096 4.9 -> 4.6 us; equal at
    // 6144 and 11008 x 4096 (kept consecutive above 16 row groups per CU at two
    // chunks per lane); 1536 x 8960 (280 chunks) 5.8 -> 6.2 us, so rows with a
    // partial run keep consecutive chunks.
    const bool il = H2 && BS == 32 && nb % 64 == 0 && (CPL >= 3 || groups <= 16 * cus);
#define ORTMI_GEMV_IL(DV)                                                                         \
    return launch_gemv4_inst<T, BS, CPL, R, DV, PRO, PAIR, false, H2, true, MRG, 1, H2 && BS == 32>( \
        A, B, S, Z, Y, N, K, nb, pro, grid, st)
    if constexpr (CPL >= 6 && H2) {
        // fp16 rows of K > 10240 (6-8 chunks per lane): two rows in flight per wave
        // (Mistral-7B's down_proj 4096 x 14336: 14.3 -> 13.1 us; 16 rows per
        // workgroup instead of 8 measured 14.7 us).
        if (il) ORTMI_GEMV_IL(2);
        if (sv) ORTMI_GEMV_INST(2, kSV, false);
        ORTMI_GEMV_INST(2, false, false);
    } else if constexpr (CPL >= 3) {
        if (il) ORTMI_GEMV_IL(1);
        if (sv) ORTMI_GEMV_INST(1, kSV, false);
        ORTMI_GEMV_INST(1, false, false);
    } else {
        if (il && !longwalk) ORTMI_GEMV_IL(2);
        if (longwalk) {
            if (sv) ORTMI_GEMV_INST(4, kSV, false);
            ORTMI_GEMV_INST(4, false, false);
        }
        if (sv) ORTMI_GEMV_INST(2, kSV, true);
        ORTMI_GEMV_INST(2, false, true);
    }
#undef ORTMI_GEMV_INST
#undef ORTMI_GEMV_IL
}

template <typename T, int BS, bool PRO = false, bool PAIR = false, bool MRG = false>
static int launch_gemv4(const T* A, const uint8_t* B, const T* S, const uint8_t* Z, T* Y, int N,
                        int K, int nb, hipStream_t st,
                        const GemvPrologue<T>& pro = GemvPrologue<T>{nullptr, nullptr, nullptr, 0.f}) {
    const int C = nb * BS / 32;
    const int cpl = (C + 63) / 64;
    if ((long)nb * BS > 2048L * (16 / (long)sizeof(T))) return -1;  // activation staging bound
    if ((size_t)N * nb * BS / 2 > 0xFFFFFF00ull) return -1;  // buffer offsets are 32-bit
    // Long walks over short rows (lm_head: 151936 x 1536): 4 rows per wave, 16
    // lanes x ceil(C/16) chunks each, so no lane idles on a 48-chunk row; cached
    // loads, ring of 2, 8 groups (32 rows) per wave: 33.6 us against 39 us with
    // a row per wave.
    constexpr int R = PAIR ? 2 : 1;
    const long units = ((long)N + R - 1) / R;
    if (units > 80L * device_cu_count() && C <= 48) {
        constexpr bool H2 = std::is_same<T, half_t>::value;
        const long grid = (units + 127) / 128;  // 4 waves x 32 rows per workgroup
        switch ((C + 15) / 16) {
            case 1: return launch_gemv4_inst<T, BS, 1, R, 2, PRO, PAIR, false, H2, false, MRG, 4>(
                        A, B, S, Z, Y, N, K, nb, pro, grid, st);
            case 2: return launch_gemv4_inst<T, BS, 2, R, 2, PRO, PAIR, false, H2, false, MRG, 4>(
                        A, B, S, Z, Y, N, K, nb, pro, grid, st);
            default: return launch_gemv4_inst<T, BS, 3, R, 2, PRO, PAIR, false, H2, false, MRG, 4>(
                        A, B, S, Z, Y, N, K, nb, pro, grid, st);
        }
    }
    switch (cpl) {
        case 1: return launch_gemv4_cpl<T, BS, 1, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
        case 2: return launch_gemv4_cpl<T, BS, 2, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
        case 3: return launch_gemv4_cpl<T, BS, 3, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
        case 4: return launch_gemv4_cpl<T, BS, 4, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
        case 5: return launch_gemv4_cpl<T, BS, 5, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
        default: break;
    }
    // fp16 activations held as pairs (16 VGPRs per chunk) also take K up to 16384
    // (the down_proj of 7B-class decoders, K = 11008 or 14336); fp32 and bf16 hold
    // 32 VGPRs per chunk and stop at 10240.
    if constexpr (std::is_same<T, half_t>::value) {
        switch (cpl) {
            case 6: return launch_gemv4_cpl<T, BS, 6, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
            case 7: return launch_gemv4_cpl<T, BS, 7, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
            case 8: return launch_gemv4_cpl<T, BS, 8, PRO, PAIR, MRG>(A, B, S, Z, Y, N, K, nb, pro, st);
            default: break;
        }
    }
    return -1;  // the caller falls back
}

// ------------------------------------------------------------- GEMM (MFMA) --

// k-steps of 64 codes. LDS rows hold 64 halfs padded to 72 (144 bytes): 16-byte
// reads of 8 consecutive rows fall in 8 different bank groups (144/16 = 9 = 1 mod 8).
constexpr int kBK = 64;
constexpr int kLdsRow = 72;

// Dequantise one 32-bit word (codes k0..k7 of a chunk) to four fp16 pairs
// (k0,k4) (k1,k5) (k2,k6) (k3,k7): (w >> 4j) & 0x000F000F | 0x6400 6400 is the
// pair (1024 + q) exactly; subtracting (1024 + zp) is exact, and the multiply by
// the scale rounds once, giving fp16((q - zp) * s).
__device__ __forceinline__ uint4 dequant_word_pairs(uint32_t w, half2_t zoff, half2_t s2) {
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t m = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        half2_t h = __builtin_bit_cast(half2_t, m);
        h = (h - zoff) * s2;
        r[j] = __builtin_bit_cast(uint32_t, h);
    }
    return make_uint4(r[0], r[1], r[2], r[3]);
}


// bf16 weights: (q - zp) is formed exactly in fp16 as above, widened and scaled
// in fp32, and rounded once to bf16 (bf16((q - zp) * s)).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
__device__ __forceinline__ uint4 dequant_word_pairs_bf16(uint32_t w, half2_t zoff, float s) {
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t m = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        const half2_t h = __builtin_bit_cast(half2_t, m) - zoff;
        const bf16x2_t v = {(__bf16)((float)h.x * s), (__bf16)((float)h.y * s)};
        r[j] = __builtin_bit_cast(uint32_t, v);
    }
    return make_uint4(r[0], r[1], r[2], r[3]);
}

// Per-element-type pieces of the MFMA GEMM: T = half_t (fp16) or uint16_t (bf16
// bits). A block's dequantisation parameters, one word of codes to four operand
// pairs, and the 32x32x16 matrix-core step.
template <typename T>
struct GemmDq {
    half2_t zoff;
    half2_t s2;  // fp16: the scale as a pair
    float s;     // bf16: the scale in fp32
};
template <typename T>
__device__ __forceinline__ GemmDq<T> gemm_dq(float zf, uint16_t sbits) {
    GemmDq<T> d;
    d.zoff = half2_t{(half_t)(1024.f + zf), (half_t)(1024.f + zf)};
    if constexpr (std::is_same<T, half_t>::value) {
        const half_t sh = __builtin_bit_cast(half_t, sbits);
        d.s2 = half2_t{sh, sh};
        d.s = 0.f;
    } else {
        d.s2 = half2_t{(half_t)0.f, (half_t)0.f};
        d.s = to_f32(sbits);
    }
    return d;
}
template <typename T>
__device__ __forceinline__ uint4 gemm_dequant(uint32_t w, const GemmDq<T>& d) {
    if constexpr (std::is_same<T, half_t>::value) return dequant_word_pairs(w, d.zoff, d.s2);
    else return dequant_word_pairs_bf16(w, d.zoff, d.s);
}
template <typename T>
__device__ __forceinline__ float16_t gemm_mfma(half8_t a, half8_t b, float16_t c) {
    if constexpr (std::is_same<T, half_t>::value)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0,
                                                       0);
}

// One k-step's loads, kept raw until they are stored to LDS (a conversion at load
// time would make the compiler wait for this load, and so for every earlier one).
template <int BM, int BN, int BS>
struct GemmStage {
    static constexpr int A_VEC = BM * kBK / 8 / 256;  // 16-byte activation vectors per thread
    uint4 a[A_VEC];
    uint4 b;         // 32 codes (one 32-code chunk of one weight row)
    // Whole registers for the small fields: packed as 16 + 8 + 8 bits, the stage
    // was carried across the loop as byte pieces, and splitting a freshly loaded
    // scale into them waited on that load (loads complete in order, so on all of
    // the stage's loads, issued only one step before) at the end of every odd
    // step, which left one step of prefetch instead of two.
    uint32_t s;      // fp16 bits of that chunk's block scale
    uint32_t z;      // zero-point byte of the block pair
    uint32_t zhi;    // 1: the block's zero point is the byte's high nibble
};

// KS = 2 splits the k-steps of a tile between two groups of 4 waves (512 threads,
// own LDS buffers, common barriers: both halves run the same number of steps),
// whose accumulators are summed through LDS at the end: 2 waves per SIMD to hide
// the load latency when the grid has only about one tile per CU.
//
// BR (weights in registers, BN = 128): the 4 waves sit side by side, each with
// all BM rows and 32 columns. Lane l of a wave loads chunk 2s + (l >> 5) of
// column (l & 31) of k-step s and dequantises it straight into its MFMA B
// operands (word kk of the chunk for sub-step kk). Only the activation tile goes
// through LDS, read at column 32 (l >> 5) + 8 kk so that both operands take the
// same codes in each k slot.
template <typename T, int BM, int BN, int BS, int KS = 1, bool SWI = false, bool BR = false>
__global__ __launch_bounds__(256 * KS) void mnb_gemm4_kernel(const T* __restrict__ A,
                                                             const uint8_t* __restrict__ B,
                                                             const T* __restrict__ S,
                                                             const uint8_t* __restrict__ Z,
                                                             T* __restrict__ Y, int M,
                                                             int N, int K, int nb, int tiles_m,
                                                             int tiles_n) {
    static_assert(sizeof(T) == 2, "fp16 or bf16 (16-bit storage)");
    // Each k-step stages BN weight rows x 2 chunks of 32 codes: one chunk per thread
    // (BN = 128) or half a chunk per thread (BN = 64).
    static_assert(BN == 128 || BN == 64, "weight tile rows");
    static_assert(KS == 1 || KS == 2, "k split");
    static_assert(!BR || BN == 128, "weights in registers: 4 waves x 32 columns");
    constexpr int WM = BR ? BM : BM / 2, WN = BR ? 32 : BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    using Stage = GemmStage<BM, BN, BS>;
    constexpr int A_VEC = Stage::A_VEC;
    __shared__ half_t sAall[KS][2][BM * kLdsRow];
    __shared__ half_t sBall[KS][2][BR ? 8 : BN * kLdsRow];
    const int half_id = KS == 2 ? (int)(threadIdx.x >> 8) : 0;
    half_t (&sA)[2][BM * kLdsRow] = sAall[half_id];
    auto& sB = sBall[half_id];

    // XCD-aware order: workgroups are dealt round-robin to the 8 XCDs; give each
    // XCD a contiguous range of tiles (m fastest) so tiles sharing weight columns
    // share that XCD's L2.
    const int nwg = gridDim.x;
    int tile = blockIdx.x;
    if (nwg % 8 == 0) tile = (blockIdx.x % 8) * (nwg / 8) + blockIdx.x / 8;
    const int tm = tile % tiles_m, tn = tile / tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
    const int wm = BR ? 0 : (wave & 1) * WM, wn = BR ? wave * 32 : (wave >> 1) * WN;
    const int Kp = nb * BS;
    const int ksteps_all = (Kp + kBK - 1) / kBK;
    // This half's k-steps: [kbase, kbase + ksteps); steps past the end read zeros.
    const int ksteps = (ksteps_all + KS - 1) / KS;
    const int kbase = half_id * ksteps;
    const int chunks = Kp / 32;
    const size_t row_bytes = (size_t)Kp / 2;
    const int zp_cols = (nb + 1) / 2;
    // Raw buffer loads with range checks: a row past M or N, or a chunk past the
    // row, reads zeros without touching memory, so no load sits behind a branch
    // and the two-step prefetch is never drained by a conservative wait. (A's
    // rows are whole 16-byte vectors: the caller guarantees K % 8 == 0.)
    const uint32_t a_end = (uint32_t)((size_t)M * K * sizeof(half_t));
    const uint32_t b_end = (uint32_t)((size_t)N * row_bytes);
    const uint32_t s_end = (uint32_t)((size_t)N * nb * sizeof(half_t));
    const uint32_t z_end = Z ? (uint32_t)((size_t)N * zp_cols) : 0u;
    const __amdgpu_buffer_rsrc_t ra =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(A), 0, (int)a_end, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rb =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(B), 0, (int)b_end, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(S), 0, (int)s_end, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rz = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(Z ? Z : B), 0, (int)z_end, kBufferWord3);

    auto gload = [&](Stage& st, int ks_local) {
        // Steps past this half's range read zeros (they may lie inside the other
        // half's range).
        const bool live = ks_local < ksteps;
        const int ks = kbase + ks_local;
        const int k0 = ks * kBK;
#pragma unroll
        for (int p = 0; p < A_VEC; ++p) {
            const int idx = tid + p * 256;
            const int r = idx >> 3, c = (idx & 7) * 8;
            const int m = m0 + r, k = k0 + c;
            const uint32_t off = (live && m < M && k < K)
                                     ? (uint32_t)(((size_t)m * K + k) * sizeof(half_t))
                                     : a_end;
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
            st.a[p] = make_uint4(v.x, v.y, v.z, v.w);
        }
        constexpr int TPR = 256 / BN;  // threads per weight row: 2 (one chunk) or 4 (half)
        // BR: column (lane & 31) of this wave's 32, chunk (lane >> 5) of the step.
        const int r = BR ? wn + (lane & 31) : tid / TPR;
        const int chunk = 2 * ks + (BR ? (lane >> 5) : (tid % TPR) * 2 / TPR);
        const int n = n0 + r;
        const bool ok = live && n < N && chunk < chunks;
        const int blk = (chunk * 32) / BS;
        if constexpr (BN == 128) {
            const uint32_t boff =
                ok ? (uint32_t)((size_t)n * row_bytes + (size_t)chunk * 16) : b_end;
            const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb, boff, 0, 0);
            st.b = make_uint4(v.x, v.y, v.z, v.w);
        } else {
            const uint32_t boff =
                ok ? (uint32_t)((size_t)n * row_bytes + (size_t)chunk * 16 + (tid & 1) * 8)
                   : b_end;
            const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rb, boff, 0, 0));
            st.b = make_uint4(v.x, v.y, 0u, 0u);
        }
        const uint32_t soff = ok ? (uint32_t)(((size_t)n * nb + blk) * sizeof(half_t)) : s_end;
        st.s = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, soff, 0, 0);  // 0 out of range
        const uint32_t zoff = ok ? (uint32_t)((size_t)n * zp_cols + blk / 2) : z_end;
        st.z = (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(rz, zoff, 0, 0);
        st.zhi = (uint32_t)(blk & 1);
    };
    auto sstore = [&](const Stage& st, int buf) {
#pragma unroll
        for (int p = 0; p < A_VEC; ++p) {
            const int idx = tid + p * 256;
            const int r = idx >> 3, c = (idx & 7) * 8;
            *reinterpret_cast<uint4*>(&sA[buf][r * kLdsRow + c]) = permute_act8(st.a[p]);
        }
        if constexpr (!BR) {
            const float zf = Z ? (float)nibble(st.z, st.zhi) : 8.f;
            const GemmDq<T> dq = gemm_dq<T>(zf, st.s);
            if constexpr (BN == 128) {
                const int r = tid >> 1, h = tid & 1;
                uint4* dst = reinterpret_cast<uint4*>(&sB[buf][r * kLdsRow + h * 32]);
                dst[0] = gemm_dequant<T>(st.b.x, dq);
                dst[1] = gemm_dequant<T>(st.b.y, dq);
                dst[2] = gemm_dequant<T>(st.b.z, dq);
                dst[3] = gemm_dequant<T>(st.b.w, dq);
            } else {
                const int r = tid >> 2, h = (tid >> 1) & 1, q = tid & 1;
                uint4* dst = reinterpret_cast<uint4*>(&sB[buf][r * kLdsRow + h * 32 + q * 16]);
                dst[0] = gemm_dequant<T>(st.b.x, dq);
                dst[1] = gemm_dequant<T>(st.b.y, dq);
            }
        }
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    // BR: the B operands of the current step, dequantised from its stage.
    uint4 bq[BR ? 4 : 1];
    auto dequant_b = [&](const Stage& st) {
        const float zf = Z ? (float)nibble(st.z, st.zhi) : 8.f;
        const GemmDq<T> dq = gemm_dq<T>(zf, st.s);
        bq[0] = gemm_dequant<T>(st.b.x, dq);
        if constexpr (BR) {
            bq[1] = gemm_dequant<T>(st.b.y, dq);
            bq[2] = gemm_dequant<T>(st.b.z, dq);
            bq[3] = gemm_dequant<T>(st.b.w, dq);
        }
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            half8_t af[TM], bf[TN];
            const int acol = BR ? 4 * lk + kk * 8 : kk * 16 + lk;
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const half8_t*>(
                    &sA[buf][(wm + i * 32 + lrow) * kLdsRow + acol]);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if constexpr (BR)
                    bf[j] = __builtin_bit_cast(half8_t, bq[kk]);
                else
                    bf[j] = *reinterpret_cast<const half8_t*>(
                        &sB[buf][(wn + j * 32 + lrow) * kLdsRow + kk * 16 + lk]);
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = gemm_mfma<T>(af[i], bf[j], acc[i][j]);
        }
    };

    // Pipeline: loads for step s are issued two steps ahead (register sets r0/r1
    // alternate), stored to the LDS buffer of step s at the end of step s-1.
    // Loads and stores past the last step are issued too (they read zeros and
    // fill a buffer nobody reads), so the loop has no branch around a load. The
    // loop runs an even number of steps (an odd count gets one all-zero step):
    // a mid-body exit made the compiler copy all accumulators every iteration.
    Stage r0, r1;
    gload(r0, 0);
    gload(r1, 1);
    sstore(r0, 0);
    __syncthreads();
    const int ksteps2 = (ksteps + 1) & ~1;
    for (int ks = 0; ks < ksteps2; ks += 2) {
        // even step ks: LDS buf 0 holds it; r1 holds step ks+1. (BR: r0's weights
        // become the B operands before r0 is reloaded.)
        if constexpr (BR) dequant_b(r0);
        gload(r0, ks + 2);
        compute(0);
        sstore(r1, 1);
        __syncthreads();
        // odd step ks+1: LDS buf 1; r0 holds step ks+2.
        if constexpr (BR) dequant_b(r1);
        gload(r1, ks + 3);
        compute(1);
        sstore(r0, 0);
        __syncthreads();
    }

    if constexpr (KS == 2) {
        // Half 1 hands its accumulators to half 0 through LDS (the loop ended on a
        // barrier, so the tile buffers are free).
        float* xch = BR ? reinterpret_cast<float*>(&sAall[0][0][0])
                        : reinterpret_cast<float*>(&sBall[0][0][0]);
        static_assert(4 * TM * TN * 16 * 64 * sizeof(float) <= (BR ? sizeof(sAall) : sizeof(sBall)),
                      "exchange space");
        if (half_id == 1) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        xch[((wave * TM * TN + i * TN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
        }
        __syncthreads();
        if (half_id == 1) return;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    acc[i][j][e] += xch[((wave * TM * TN + i * TN + j) * 16 + e) * 64 + lane];
    }
    // D layout of a 32x32 MFMA: lane holds column (lane & 31); accumulator e holds
    // row 8*(e/4) + 4*(lane/32) + (e%4).
    if constexpr (SWI) {
        // Interleaved gate/up columns (2i, 2i+1) sit in lanes (2l, 2l+1): the even
        // lane takes its partner's value and writes column i of the [M, N/2] output,
        // (g * sigmoid(g)) * u with each op rounded to fp16 as the unfused ops store.
        const int Nh = N / 2;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int n = n0 + wn + j * 32 + (lane & 31);
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float y = round_to<T>(acc[i][j][e]);
                    const float partner = dpp_mov<0xB1>(y);  // quad_perm [1,0,3,2]
                    const int m = m0 + wm + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                    if ((lane & 1) == 0 && m < M && n < N) {
                        const float sig = round_to<T>(1.0f / (1.0f + __expf(-y)));
                        Y[(size_t)m * Nh + n / 2] = from_f32<T>(round_to<T>(y * sig) * partner);
                    }
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn + j * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                if (m < M && n < N) Y[(size_t)m * N + n] = from_f32<T>(acc[i][j][e]);
            }
        }
}

template <typename T, int BM, int BN, int BS, int KS = 1, bool SWI = false, bool BR = false>
static int launch_gemm4(const T* A, const uint8_t* B, const T* S, const uint8_t* Z,
                        T* Y, int M, int N, int K, int nb, hipStream_t st) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    hipLaunchKernelGGL((mnb_gemm4_kernel<T, BM, BN, BS, KS, SWI, BR>), dim3(tiles_m * tiles_n),
                       dim3(256 * KS), 0, st, A, B, S, Z, Y, M, N, K, nb, tiles_m, tiles_n);
    return check_launch("mnb_gemm4");
}

template <typename T, int BS, bool SWI = false>
static int dispatch_gemm4(const T* A, const uint8_t* B, const T* S, const uint8_t* Z,
                          T* Y, int M, int N, int K, int nb, hipStream_t st) {
    // 128x128 tiles once they fill the CUs twice over; below that, the k-steps are
    // split over two wave groups, with 64x128 tiles while those still give every
    // CU a tile and 64x64 tiles under that (M=512 on MI355X: K=N=4096 41.6 us
    // with 64x128; N=1536 K=8960 66.4 -> 49.7 us, N=2048 K=1536 15.1 -> 11.5 us
    // with 64x64).
    const int cus = device_cu_count();
    const long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    // 128x128 tiles take their weights in registers (gate/up 512x17920x1536:
    // 52-54 -> 46-47 us); at 64x128 the LDS form measured equal or faster.
    if (big >= 2L * cus)
        return launch_gemm4<T, 128, 128, BS, 1, SWI, true>(A, B, S, Z, Y, M, N, K, nb, st);
    const long mid = (long)((M + 63) / 64) * ((N + 127) / 128);
    if (mid >= cus) return launch_gemm4<T, 64, 128, BS, 2, SWI>(A, B, S, Z, Y, M, N, K, nb, st);
    return launch_gemm4<T, 64, 64, BS, 2, SWI>(A, B, S, Z, Y, M, N, K, nb, st);
}

// ----------------------------------------------------------------- generic --

// Any bits/block/dtype: 64x64 output tile, 256 threads, 4x4 outputs per thread,
// fp32 dequantisation of a 64x32 weight tile into LDS.
template <typename T>
__global__ __launch_bounds__(256) void mnb_generic_kernel(const T* __restrict__ A,
                                                          const uint8_t* __restrict__ B,
                                                          const T* __restrict__ S,
                                                          const uint8_t* __restrict__ Z,
                                                          T* __restrict__ Y, int M, int N, int K,
                                                          int nb, int bits, int bs) {
    __shared__ float sA[64][33];
    __shared__ float sW[64][33];
    const int tid = threadIdx.x;
    const int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    const int tr = tid / 16, tc = tid % 16;
    const size_t blob = (size_t)bs * bits / 8;
    const int zp_cols = bits == 4 ? (nb + 1) / 2 : nb;
    const int zdef = 1 << (bits - 1);
    float acc[4][4] = {};
    for (int k0 = 0; k0 < K; k0 += 32) {
        for (int i = tid; i < 64 * 32; i += 256) {
            const int r = i / 32, c = i % 32;
            const int m = m0 + r, k = k0 + c;
            sA[r][c] = (m < M && k < K) ? to_f32(A[(size_t)m * K + k]) : 0.f;
            const int n = n0 + r;
            float wv = 0.f;
            if (n < N && k < K) {
                const int blk = k / bs, within = k % bs;
                int q, z;
                if (bits == 4) {
                    const uint8_t byte = B[((size_t)n * nb + blk) * blob + within / 2];
                    q = nibble(byte, within & 1);
                    z = Z ? nibble(Z[(size_t)n * zp_cols + blk / 2], blk & 1) : zdef;
                } else {
                    q = B[((size_t)n * nb + blk) * blob + within];
                    z = Z ? Z[(size_t)n * zp_cols + blk] : zdef;
                }
                wv = (float)(q - z) * to_f32(S[(size_t)n * nb + blk]);
            }
            sW[r][c] = wv;
        }
        __syncthreads();
#pragma unroll 8
        for (int kk = 0; kk < 32; ++kk) {
            float av[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = sA[tr * 4 + i][kk];
#pragma unroll
            for (int j = 0; j < 4; ++j) wv[j] = sW[tc * 4 + j][kk];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], wv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int m = m0 + tr * 4 + i, n = n0 + tc * 4 + j;
            if (m < M && n < N) Y[(size_t)m * N + n] = from_f32<T>(acc[i][j]);
        }
}

template <typename T>
static int launch_generic(const T* A, const uint8_t* B, const T* S, const uint8_t* Z, T* Y, int M,
                          int N, int K, int nb, int bits, int bs, hipStream_t st) {
    dim3 grid((N + 63) / 64, (M + 63) / 64);
    hipLaunchKernelGGL((mnb_generic_kernel<T>), grid, dim3(256), 0, st, A, B, S, Z, Y, M, N, K, nb,
                       bits, bs);
    return check_launch("mnb_generic");
}

template <typename T>
static int run_mnb(const void* A, const uint8_t* B, const void* S, const uint8_t* Z, void* Y,
                   int M, int N, int K, int bits, int bs, hipStream_t st) {
    const int nb = (K + bs - 1) / bs;
    const T* a = static_cast<const T*>(A);
    const T* s = static_cast<const T*>(S);
    T* y = static_cast<T*>(Y);
    const bool aligned = (reinterpret_cast<uintptr_t>(B) % 16) == 0;
    const bool fast_form = bits == 4 && (bs == 32 || bs == 64 || bs == 128) && aligned;
    const size_t kmax = std::is_same<T, half_t>::value ? 16384 : 10240;
    if (fast_form && M == 1 && (size_t)nb * bs <= kmax) {
        int rc = -1;
        if (bs == 32) rc = launch_gemv4<T, 32>(a, B, s, Z, y, N, K, nb, st);
        if (bs == 64) rc = launch_gemv4<T, 64>(a, B, s, Z, y, N, K, nb, st);
        if (bs == 128) rc = launch_gemv4<T, 128>(a, B, s, Z, y, N, K, nb, st);
        if (rc >= 0) return rc;
    }
    if constexpr (sizeof(T) == 2) {  // fp16 and bf16 prefill on the matrix cores
        const bool a_aligned = (reinterpret_cast<uintptr_t>(A) % 16) == 0 && K % 8 == 0;
        const bool fits32 = (size_t)M * K * 2 <= 0xFFFFFF00ull &&
                            (size_t)N * nb * bs / 2 <= 0xFFFFFF00ull;  // 32-bit buffer offsets
        if (fast_form && M > 1 && a_aligned && fits32) {
            if (bs == 32) return dispatch_gemm4<T, 32>(a, B, s, Z, y, M, N, K, nb, st);
            if (bs == 64) return dispatch_gemm4<T, 64>(a, B, s, Z, y, M, N, K, nb, st);
            if (bs == 128) return dispatch_gemm4<T, 128>(a, B, s, Z, y, M, N, K, nb, st);
        }
    }
    return launch_generic<T>(a, B, s, Z, y, M, N, K, nb, bits, bs, st);
}

}  // namespace ortmi

using namespace ortmi;

namespace ortmi {
template <typename T, bool PRO, bool PAIR>
static int run_fused_gemv(const void* x, const void* skip, const void* gamma, float eps,
                          void* residual, const uint8_t* B, const void* S, const uint8_t* Z,
                          void* Y, int N, int K, int bs, hipStream_t st) {
    const int nb = (K + bs - 1) / bs;
    GemvPrologue<T> pro{static_cast<const T*>(skip), static_cast<const T*>(gamma),
                        static_cast<T*>(residual), eps};
    const T* a = static_cast<const T*>(x);
    const T* s = static_cast<const T*>(S);
    T* y = static_cast<T*>(Y);
    if (bs == 32) return launch_gemv4<T, 32, PRO, PAIR>(a, B, s, Z, y, N, K, nb, st, pro);
    if (bs == 64) return launch_gemv4<T, 64, PRO, PAIR>(a, B, s, Z, y, N, K, nb, st, pro);
    return launch_gemv4<T, 128, PRO, PAIR>(a, B, s, Z, y, N, K, nb, st, pro);
}

template <typename T>
static int dispatch_fused_gemv(const void* x, const void* skip, const void* gamma, float eps,
                               void* residual, const uint8_t* B, const void* S,
                               const uint8_t* Z, void* Y, int N, int K, int bs, bool norm,
                               bool pair, hipStream_t st) {
    if (norm && pair)
        return run_fused_gemv<T, true, true>(x, skip, gamma, eps, residual, B, S, Z, Y, N, K, bs, st);
    if (norm)
        return run_fused_gemv<T, true, false>(x, skip, gamma, eps, residual, B, S, Z, Y, N, K, bs, st);
    if (pair)
        return run_fused_gemv<T, false, true>(x, skip, gamma, eps, residual, B, S, Z, Y, N, K, bs, st);
    return run_fused_gemv<T, false, false>(x, skip, gamma, eps, residual, B, S, Z, Y, N, K, bs, st);
}
}  // namespace ortmi

extern "C" int ortmi_matmul_nbits_decode_fused(const void* x, const void* skip, const void* gamma,
                                               float epsilon, void* residual, const uint8_t* B,
                                               const void* scales, const uint8_t* zero_points,
                                               void* Y, int64_t N, int64_t K, int64_t block_size,
                                               int32_t flags, int32_t dtype, void* stream) {
    const bool norm = (flags & ORTMI_FUSE_RMS_NORM) != 0;
    const bool pair = (flags & ORTMI_FUSE_SWIGLU_PAIRS) != 0;
    ORTMI_REQUIRE((flags & ~(ORTMI_FUSE_RMS_NORM | ORTMI_FUSE_SWIGLU_PAIRS)) == 0,
                  "MatMulNBits fused: unknown flags");
    ORTMI_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128,
                  "MatMulNBits fused: block_size must be 32, 64 or 128");
    ORTMI_REQUIRE(N > 0 && K > 0 && N < (1LL << 31), "MatMulNBits fused: bad shape");
    ORTMI_REQUIRE(!pair || N % 2 == 0, "MatMulNBits fused: SwiGLU pairs need an even N");
    ORTMI_REQUIRE(x && B && scales && Y, "MatMulNBits fused: null tensor");
    ORTMI_REQUIRE(!norm || gamma, "MatMulNBits fused: the norm needs gamma");
    ORTMI_REQUIRE(!residual || (norm && skip), "MatMulNBits fused: residual needs the skip norm");
    ORTMI_REQUIRE((reinterpret_cast<uintptr_t>(B) & 15) == 0,
                  "MatMulNBits fused: B must be 16-byte aligned");
    const int64_t nb = (K + block_size - 1) / block_size;
    const int64_t limit = 2048LL * (dtype == ORTMI_F32 ? 4 : 8);
    ORTMI_REQUIRE(nb * block_size <= std::min<int64_t>(limit, dtype == ORTMI_F16 ? 16384 : 10240),
                  "MatMulNBits fused: K too large for the decode kernel");
    hipStream_t st = as_stream(stream);
    int rc;
    switch (dtype) {
        case ORTMI_F16:
            rc = dispatch_fused_gemv<half_t>(x, skip, gamma, epsilon, residual, B, scales,
                                             zero_points, Y, (int)N, (int)K, (int)block_size, norm,
                                             pair, st);
            break;
        case ORTMI_BF16:
            rc = dispatch_fused_gemv<uint16_t>(x, skip, gamma, epsilon, residual, B, scales,
                                               zero_points, Y, (int)N, (int)K, (int)block_size,
                                               norm, pair, st);
            break;
        default:
            return fail(ORTMI_E_INVALID, "MatMulNBits fused: fp16 or bf16 activations only");
    }
    // The launcher declines shapes beyond its staging or 32-bit buffer range.
    if (rc < 0) return fail(ORTMI_E_INVALID, "MatMulNBits fused: shape has no decode kernel");
    return rc;
}

namespace ortmi {
template <typename T>
static int run_merge_gemv(const float* part, int splits, int hd, const uint8_t* B, const void* S,
                          const uint8_t* Z, void* Y, int N, int K, int bs, hipStream_t st) {
    const int nb = (K + bs - 1) / bs;
    GemvPrologue<T> pro{nullptr, nullptr, nullptr, 0.f, part, splits, hd};
    const T* s = static_cast<const T*>(S);
    T* y = static_cast<T*>(Y);
    if (bs == 32) return launch_gemv4<T, 32, false, false, true>(nullptr, B, s, Z, y, N, K, nb, st, pro);
    if (bs == 64) return launch_gemv4<T, 64, false, false, true>(nullptr, B, s, Z, y, N, K, nb, st, pro);
    return launch_gemv4<T, 128, false, false, true>(nullptr, B, s, Z, y, N, K, nb, st, pro);
}
}  // namespace ortmi

extern "C" int ortmi_matmul_nbits_decode_merge(const float* partials, int64_t splits,
                                               int64_t head_size, const uint8_t* B,
                                               const void* scales, const uint8_t* zero_points,
                                               void* Y, int64_t N, int64_t K, int64_t block_size,
                                               int32_t dtype, void* stream) {
    ORTMI_REQUIRE(partials && B && scales && Y, "MatMulNBits merge: null tensor");
    ORTMI_REQUIRE(splits >= 1 && splits <= 4096, "MatMulNBits merge: bad split count");
    ORTMI_REQUIRE(head_size == 64 || head_size == 128,
                  "MatMulNBits merge: head_size must be 64 or 128");
    ORTMI_REQUIRE(K > 0 && K % head_size == 0 && N > 0 && N < (1LL << 31),
                  "MatMulNBits merge: K must be a whole number of heads");
    ORTMI_REQUIRE(block_size == 32 || block_size == 64 || block_size == 128,
                  "MatMulNBits merge: block_size must be 32, 64 or 128");
    ORTMI_REQUIRE((reinterpret_cast<uintptr_t>(B) & 15) == 0,
                  "MatMulNBits merge: B must be 16-byte aligned");
    const int64_t nb = (K + block_size - 1) / block_size;
    ORTMI_REQUIRE(nb * block_size <= 10240, "MatMulNBits merge: K too large for the decode kernel");
    ORTMI_REQUIRE((reinterpret_cast<uintptr_t>(partials) & 15) == 0,
                  "MatMulNBits merge: partials must be 16-byte aligned");
    const size_t stage = (size_t)nb * block_size * (dtype == ORTMI_F16 ? 2 : 4);
    if ((K / head_size) * splits * (head_size + 2) > kDecodeMergeMaxFloats ||
        gemv_merge_bytes((int)K, (int)head_size, (int)splits) + stage > 65536)
        return fail(ORTMI_E_INVALID, "MatMulNBits merge: too many split partials for one workgroup");
    hipStream_t st = as_stream(stream);
    int rc = -1;
    if (dtype == ORTMI_F16)
        rc = run_merge_gemv<half_t>(partials, (int)splits, (int)head_size, B, scales, zero_points,
                                    Y, (int)N, (int)K, (int)block_size, st);
    else if (dtype == ORTMI_BF16)
        rc = run_merge_gemv<uint16_t>(partials, (int)splits, (int)head_size, B, scales,
                                      zero_points, Y, (int)N, (int)K, (int)block_size, st);
    else
        return fail(ORTMI_E_INVALID, "MatMulNBits merge: fp16 or bf16 activations only");
    if (rc < 0) return fail(ORTMI_E_INVALID, "MatMulNBits merge: shape has no decode kernel");
    return rc;
}

extern "C" int ortmi_matmul_nbits_swiglu_pairs(const void* A, const uint8_t* B,
                                               const void* scales, const uint8_t* zero_points,
                                               void* Y, int64_t M, int64_t N, int64_t K,
                                               int64_t block_size, int32_t dtype, void* stream) {
    ORTMI_REQUIRE(M >= 0 && N >= 0 && K > 0 && N % 2 == 0 && M < (1LL << 31) &&
                      N < (1LL << 31) && K < (1LL << 31),
                  "MatMulNBits SwiGLU pairs: bad shape (N must be even)");
    if (M == 0 || N == 0) return ORTMI_OK;
    ORTMI_REQUIRE(A && B && scales && Y, "MatMulNBits SwiGLU pairs: null tensor");
    const int nb = (int)((K + block_size - 1) / block_size);
    const bool ok = dtype == ORTMI_F16 && (block_size == 32 || block_size == 64 ||
                                           block_size == 128) &&
                    (reinterpret_cast<uintptr_t>(B) % 16) == 0 &&
                    (reinterpret_cast<uintptr_t>(A) % 16) == 0 && K % 8 == 0 &&
                    (size_t)M * K * 2 <= 0xFFFFFF00ull &&
                    (size_t)N * nb * block_size / 2 <= 0xFFFFFF00ull;
    if (!ok)
        return fail(ORTMI_E_INVALID,
                    "MatMulNBits SwiGLU pairs: needs fp16, 4-bit block 32/64/128, 16-byte "
                    "aligned A and B, K % 8 == 0");
    const half_t* a = static_cast<const half_t*>(A);
    const half_t* s = static_cast<const half_t*>(scales);
    half_t* y = static_cast<half_t*>(Y);
    hipStream_t st = as_stream(stream);
    const int m = (int)M, n = (int)N, k = (int)K;
    if (block_size == 32)
        return dispatch_gemm4<half_t, 32, true>(a, B, s, zero_points, y, m, n, k, nb, st);
    if (block_size == 64)
        return dispatch_gemm4<half_t, 64, true>(a, B, s, zero_points, y, m, n, k, nb, st);
    return dispatch_gemm4<half_t, 128, true>(a, B, s, zero_points, y, m, n, k, nb, st);
}

extern "C" int ortmi_matmul_nbits(const void* A, const uint8_t* B, const void* scales,
                                  const uint8_t* zero_points, void* Y, int64_t M, int64_t N,
                                  int64_t K, int64_t bits, int64_t block_size, int32_t dtype,
                                  void* stream) {
    // Claim contract of rust/src/ops/quant.rs:1655-1711 plus shape checks.
    ORTMI_REQUIRE(bits == 4 || bits == 8, "MatMulNBits: only 4-bit and 8-bit weights are supported");
    ORTMI_REQUIRE(block_size == 16 || block_size == 32 || block_size == 64 || block_size == 128,
                  "MatMulNBits: block_size must be 16, 32, 64, or 128");
    ORTMI_REQUIRE(M >= 0 && N >= 0 && K >= 0, "MatMulNBits: negative dimension");
    ORTMI_REQUIRE(M < (1LL << 31) && N < (1LL << 31) && K < (1LL << 31),
                  "MatMulNBits: dimension too large");
    if (M == 0 || N == 0) return ORTMI_OK;
    ORTMI_REQUIRE(K > 0, "MatMulNBits: K must be positive");
    ORTMI_REQUIRE(A && B && scales && Y, "MatMulNBits: null tensor");
    hipStream_t st = as_stream(stream);
    switch (dtype) {
        case ORTMI_F32:
            return run_mnb<float>(A, B, scales, zero_points, Y, (int)M, (int)N, (int)K, (int)bits,
                                  (int)block_size, st);
        case ORTMI_F16:
            return run_mnb<half_t>(A, B, scales, zero_points, Y, (int)M, (int)N, (int)K, (int)bits,
                                   (int)block_size, st);
        case ORTMI_BF16:
            return run_mnb<uint16_t>(A, B, scales, zero_points, Y, (int)M, (int)N, (int)K,
                                     (int)bits, (int)block_size, st);
        default:
            return fail(ORTMI_E_INVALID,
                        "MatMulNBits: activation/scales must be float (fp32/fp16/bf16)");
    }
}

// --------------------------------------------------- GatherBlockQuantized --

namespace ortmi {

// Rows of an int4 block-quantised table gathered by index: data [V, D/2] (two
// codes per byte, low nibble first, the MatMulNBits row layout), scales
// [V, ceil(D/block)], optional packed zero points [V, ceil(nblocks/2)] (low nibble
// = even block; 8 when absent). out[i, k] = (q - zp) * scale in fp32, rounded
// once to the output type. One thread per data byte (two codes); an index outside
// [-V, V) yields a zero row (the host reports no error from device data).
template <typename T, typename I>
__global__ void gbq_kernel(const uint8_t* __restrict__ data, const T* __restrict__ scales,
                           const uint8_t* __restrict__ zp, const I* __restrict__ idx,
                           T* __restrict__ out, int64_t n_idx, int64_t V, int D, int block) {
    const int bytes = D / 2;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n_idx * bytes) return;
    const int64_t i = t / bytes;
    const int j = (int)(t % bytes);
    int64_t row = (int64_t)idx[i];
    if (row < 0) row += V;
    const bool ok = row >= 0 && row < V;
    const int nb = (D + block - 1) / block;
    const int zcols = (nb + 1) / 2;
    float v[2] = {0.f, 0.f};
    if (ok) {
        const uint8_t b = data[row * bytes + j];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = 2 * j + h;
            const int blk = k / block;
            const float s = to_f32(scales[row * nb + blk]);
            const int z = zp ? nibble(zp[row * zcols + blk / 2], blk & 1) : 8;
            v[h] = (float)(nibble(b, h) - z) * s;
        }
    }
    out[i * D + 2 * j] = from_f32<T>(v[0]);
    out[i * D + 2 * j + 1] = from_f32<T>(v[1]);
}

template <typename T>
static int launch_gbq(const uint8_t* data, const void* scales, const uint8_t* zp,
                      const void* idx, int idx_is_i64, void* out, int64_t n_idx, int64_t V,
                      int64_t D, int64_t block, hipStream_t st) {
    const int64_t threads = n_idx * (D / 2);
    if (threads == 0) return ORTMI_OK;
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (idx_is_i64)
        hipLaunchKernelGGL((gbq_kernel<T, int64_t>), dim3(grid), dim3(256), 0, st, data,
                           static_cast<const T*>(scales), zp, static_cast<const int64_t*>(idx),
                           static_cast<T*>(out), n_idx, V, (int)D, (int)block);
    else
        hipLaunchKernelGGL((gbq_kernel<T, int32_t>), dim3(grid), dim3(256), 0, st, data,
                           static_cast<const T*>(scales), zp, static_cast<const int32_t*>(idx),
                           static_cast<T*>(out), n_idx, V, (int)D, (int)block);
    return check_launch("gather_block_quantized");
}

}  // namespace ortmi

extern "C" int ortmi_gather_block_quantized(const uint8_t* data, const void* scales,
                                            const uint8_t* zero_points, const void* indices,
                                            int32_t indices_are_int64, void* output,
                                            int64_t num_indices, int64_t rows, int64_t D,
                                            int64_t block_size, int64_t bits, int32_t dtype,
                                            void* stream) {
    // Claim contract of rust/src/ops/quant.rs:1713-1749: 4-bit codes, gather axis 0,
    // quantize axis 1, block >= 16; data/zero points uint8, scales = output dtype.
    ORTMI_REQUIRE(bits == 4, "GatherBlockQuantized: only 4-bit data is supported");
    ORTMI_REQUIRE(block_size >= 16, "GatherBlockQuantized: block_size must be at least 16");
    ORTMI_REQUIRE(num_indices >= 0 && rows > 0 && D > 0 && D % 2 == 0 && D < (1LL << 30),
                  "GatherBlockQuantized: bad shape");
    ORTMI_REQUIRE(num_indices == 0 || (data && scales && indices && output),
                  "GatherBlockQuantized: null tensor");
    hipStream_t st = as_stream(stream);
    switch (dtype) {
        case ORTMI_F32:
            return launch_gbq<float>(data, scales, zero_points, indices, indices_are_int64, output,
                                     num_indices, rows, D, block_size, st);
        case ORTMI_F16:
            return launch_gbq<half_t>(data, scales, zero_points, indices, indices_are_int64,
                                      output, num_indices, rows, D, block_size, st);
        case ORTMI_BF16:
            return launch_gbq<uint16_t>(data, scales, zero_points, indices, indices_are_int64,
                                        output, num_indices, rows, D, block_size, st);
        default:
            return fail(ORTMI_E_INVALID, "GatherBlockQuantized: scales must be fp32, fp16 or bf16");
    }
}
