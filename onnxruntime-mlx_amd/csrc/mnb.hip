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
//    lane owns fixed 32-code chunks of K and keeps the matching activations in
//    VGPRs (staged once per workgroup through LDS), then streams rows of B with
//    128-bit loads (a wave reads 1 KiB contiguous per instruction). Zero points
//    are folded as s*(sum(a*q) - zp*sum(a)), so the inner loop is one
//    byte-convert + one FMA per code.
//  * mnb_gemm4  - prefill (M > 1, fp16), bits 4, bs in {32, 64, 128}. MFMA
//    v_mfma_f32_32x32x16_f16: the weight tile is dequantised to fp16 in LDS
//    (fp16((q - zp) * s), one rounding) and the activation tile is staged in LDS;
//    fp32 accumulation, one rounding of Y.
//  * mnb_generic - every other form (bits 8, bs 16, fp32/bf16 prefill): fp32
//    dequant to LDS and a VALU tile product.
#include "common.h"

namespace ortmi {

// -------------------------------------------------------------- GEMV (M=1) --

// Dot product of 32 activations with the 32 4-bit codes of one 16-byte chunk.
// Code i of the chunk is nibble (i & 1) of byte i/2, i.e. bits [4i, 4i+4) of the
// little-endian 128-bit word.
__device__ __forceinline__ float dot32_codes(const float* a, uint4 w) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = words[i] & 0x0F0F0F0Fu;         // codes 8i+0,2,4,6
        const uint32_t hi = (words[i] >> 4) & 0x0F0F0F0Fu;  // codes 8i+1,3,5,7
        const float* ai = a + 8 * i;
        d0 = fmaf(ai[0], (float)(lo & 0xffu), d0);
        d1 = fmaf(ai[1], (float)(hi & 0xffu), d1);
        d0 = fmaf(ai[2], (float)((lo >> 8) & 0xffu), d0);
        d1 = fmaf(ai[3], (float)((hi >> 8) & 0xffu), d1);
        d0 = fmaf(ai[4], (float)((lo >> 16) & 0xffu), d0);
        d1 = fmaf(ai[5], (float)((hi >> 16) & 0xffu), d1);
        d0 = fmaf(ai[6], (float)(lo >> 24), d0);
        d1 = fmaf(ai[7], (float)(hi >> 24), d1);
    }
    return d0 + d1;
}

template <typename T, int BS, int BPL, int R>
__global__ __launch_bounds__(256) void mnb_gemv4_kernel(const T* __restrict__ A,
                                                        const uint8_t* __restrict__ B,
                                                        const T* __restrict__ S,
                                                        const uint8_t* __restrict__ Z,
                                                        T* __restrict__ Y, int N, int K,
                                                        int nb) {
    extern __shared__ float sA[];
    const int Kp = nb * BS;
    const int C = Kp / 32;  // 32-code chunks per row
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int waves_total = gridDim.x * 4;
    const int gw = blockIdx.x * 4 + wave;
    const size_t row_bytes = (size_t)Kp / 2;
    const int zp_cols = (nb + 1) / 2;

    // Issue the first row group's weight loads before staging A so the HBM
    // latency overlaps the activation staging.
    uint4 w[R][BPL];
    auto load_group = [&](int n0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int j = 0; j < BPL; ++j) {
                const int n = n0 + r, c = lane + 64 * j;
                if (n < N && c < C) {
                    const u32x4_t v = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4_t*>(B + (size_t)n * row_bytes) + c);
                    w[r][j] = make_uint4(v.x, v.y, v.z, v.w);
                } else {
                    w[r][j] = make_uint4(0, 0, 0, 0);
                }
            }
    };
    int n0 = gw * R;
    if (n0 < N) load_group(n0);

    for (int k = threadIdx.x; k < Kp; k += 256) sA[k] = k < K ? to_f32(A[k]) : 0.f;
    __syncthreads();

    float a[BPL][32];
    float asum[BPL];
#pragma unroll
    for (int j = 0; j < BPL; ++j) {
        const int c = lane + 64 * j;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            a[j][i] = c < C ? sA[32 * c + i] : 0.f;
            s += a[j][i];
        }
        asum[j] = s;
    }

    for (; n0 < N; n0 += waves_total * R) {
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int n = n0 + r;
            float total = 0.f;
#pragma unroll
            for (int j = 0; j < BPL; ++j) {
                const int c = lane + 64 * j;
                if (n < N && c < C) {
                    const int blk = (32 * c) / BS;
                    const float s = to_f32(S[(size_t)n * nb + blk]);
                    const float z = Z ? (float)nibble(Z[(size_t)n * zp_cols + blk / 2], blk & 1)
                                      : 8.f;
                    const float d = dot32_codes(a[j], w[r][j]);
                    total = fmaf(s, d - z * asum[j], total);
                }
            }
            acc[r] = total;
        }
        const int next = n0 + waves_total * R;
        if (next < N) load_group(next);
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = wave_sum(acc[r]);
        if (lane < R) {
            float v = acc[0];
#pragma unroll
            for (int r = 1; r < R; ++r)
                if (lane == r) v = acc[r];
            if (n0 + lane < N) Y[n0 + lane] = from_f32<T>(v);
        }
    }
}

template <typename T, int BS, int BPL>
static int launch_gemv4_bpl(const T* A, const uint8_t* B, const T* S, const uint8_t* Z, T* Y,
                            int N, int K, int nb, hipStream_t st) {
    constexpr int R = BPL == 1 ? 8 : (BPL == 2 ? 4 : 2);
    const int Kp = nb * BS;
    const int groups = (N + R - 1) / R;
    int grid = (groups + 3) / 4;
    const int cap = device_cu_count() * 4;
    if (grid > cap) grid = cap;
    hipLaunchKernelGGL((mnb_gemv4_kernel<T, BS, BPL, R>), dim3(grid), dim3(256),
                       (size_t)Kp * sizeof(float), st, A, B, S, Z, Y, N, K, nb);
    return check_launch("mnb_gemv4");
}

template <typename T, int BS>
static int launch_gemv4(const T* A, const uint8_t* B, const T* S, const uint8_t* Z, T* Y, int N,
                        int K, int nb, hipStream_t st) {
    const int C = nb * BS / 32;
    const int bpl = (C + 63) / 64;
    switch (bpl) {
        case 1: return launch_gemv4_bpl<T, BS, 1>(A, B, S, Z, Y, N, K, nb, st);
        case 2: return launch_gemv4_bpl<T, BS, 2>(A, B, S, Z, Y, N, K, nb, st);
        case 3: return launch_gemv4_bpl<T, BS, 3>(A, B, S, Z, Y, N, K, nb, st);
        case 4: return launch_gemv4_bpl<T, BS, 4>(A, B, S, Z, Y, N, K, nb, st);
        case 5: return launch_gemv4_bpl<T, BS, 5>(A, B, S, Z, Y, N, K, nb, st);
        case 6: return launch_gemv4_bpl<T, BS, 6>(A, B, S, Z, Y, N, K, nb, st);
        case 7: return launch_gemv4_bpl<T, BS, 7>(A, B, S, Z, Y, N, K, nb, st);
        case 8: return launch_gemv4_bpl<T, BS, 8>(A, B, S, Z, Y, N, K, nb, st);
        default: return -1;  // caller falls back
    }
}

// ------------------------------------------------------------- GEMM (MFMA) --

// LDS rows are 32 halfs of data padded to 40 (80 bytes): 8 consecutive lanes
// reading 16 bytes at row stride 80 hit 8 disjoint 16-byte bank groups.
constexpr int kLdsRow = 40;

template <int BM, int BN, int BS>
__global__ __launch_bounds__(256) void mnb_gemm4_kernel(const half_t* __restrict__ A,
                                                        const uint8_t* __restrict__ B,
                                                        const half_t* __restrict__ S,
                                                        const uint8_t* __restrict__ Z,
                                                        half_t* __restrict__ Y, int M, int N,
                                                        int K, int nb, int tiles_m,
                                                        int tiles_n) {
    // Wave layout 2 x 2; each wave owns a (BM/2) x (BN/2) block of 32x32 MFMA tiles.
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int TM = WM / 32, TN = WN / 32;
    __shared__ half_t sA[2][BM * kLdsRow];
    __shared__ half_t sB[2][BN * kLdsRow];

    // XCD-aware tile order: workgroups are dealt round-robin to the 8 XCDs, so
    // remap so that each XCD receives a contiguous range of tiles (tiles that
    // share activation rows then share that XCD's L2).
    const int nwg = gridDim.x;
    const int bid = blockIdx.x;
    int tile = bid;
    if (nwg % 8 == 0) tile = (bid % 8) * (nwg / 8) + bid / 8;
    const int tm = tile % tiles_m;
    const int tn = tile / tiles_m;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = (wave & 1) * WM, wn = (wave >> 1) * WN;
    const int Kp = nb * BS;
    const int ksteps = Kp / 32;
    const size_t row_bytes = (size_t)Kp / 2;
    const int zp_cols = (nb + 1) / 2;

    // Global->register staging assignments.
    // A: BM x 32 halfs = BM*64 bytes; 16 bytes per thread per pass.
    constexpr int A_PASSES = (BM * 4) / 256;
    // B: BN rows x 16 bytes of codes; two threads per row, 8 bytes each.
    constexpr int B_PASSES = (BN * 2) / 256;
    uint4 ra[A_PASSES];
    uint2 rb[B_PASSES];
    float rs[B_PASSES], rz[B_PASSES];

    auto gload = [&](int ks) {
        const int k0 = ks * 32;
#pragma unroll
        for (int p = 0; p < A_PASSES; ++p) {
            const int idx = tid + p * 256;
            const int r = idx >> 2, c = (idx & 3) * 8;
            const int m = m0 + r, k = k0 + c;
            if (m < M && k + 8 <= K) {
                ra[p] = *reinterpret_cast<const uint4*>(A + (size_t)m * K + k);
            } else if (m < M && k < K) {
                half_t t[8];
                for (int i = 0; i < 8; ++i) t[i] = (k + i < K) ? A[(size_t)m * K + k + i] : (half_t)0;
                ra[p] = *reinterpret_cast<uint4*>(t);
            } else {
                ra[p] = make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int p = 0; p < B_PASSES; ++p) {
            const int idx = tid + p * 256;
            const int r = idx >> 1, h = idx & 1;
            const int n = n0 + r;
            if (n < N) {
                rb[p] = *reinterpret_cast<const uint2*>(B + (size_t)n * row_bytes + ks * 16 + h * 8);
                const int blk = k0 / BS;
                rs[p] = (float)S[(size_t)n * nb + blk];
                rz[p] = Z ? (float)nibble(Z[(size_t)n * zp_cols + blk / 2], blk & 1) : 8.f;
            } else {
                rb[p] = make_uint2(0, 0);
                rs[p] = 0.f;
                rz[p] = 0.f;
            }
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < A_PASSES; ++p) {
            const int idx = tid + p * 256;
            const int r = idx >> 2, c = (idx & 3) * 8;
            *reinterpret_cast<uint4*>(&sA[buf][r * kLdsRow + c]) = ra[p];
        }
#pragma unroll
        for (int p = 0; p < B_PASSES; ++p) {
            const int idx = tid + p * 256;
            const int r = idx >> 1, h = idx & 1;
            const uint32_t wds[2] = {rb[p].x, rb[p].y};
            half_t out[16];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float q = (float)((wds[i] >> (4 * j)) & 0xfu);
                    out[i * 8 + j] = (half_t)((q - rz[p]) * rs[p]);
                }
            uint4* dst = reinterpret_cast<uint4*>(&sB[buf][r * kLdsRow + h * 16]);
            dst[0] = reinterpret_cast<uint4*>(out)[0];
            dst[1] = reinterpret_cast<uint4*>(out)[1];
        }
    };

    float16_t acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    gload(0);
    sstore(0);
    __syncthreads();
    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    for (int ks = 0; ks < ksteps; ++ks) {
        const int buf = ks & 1;
        if (ks + 1 < ksteps) gload(ks + 1);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            half8_t af[TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                af[i] = *reinterpret_cast<const half8_t*>(
                    &sA[buf][(wm + i * 32 + lrow) * kLdsRow + kk * 16 + lk]);
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bf[j] = *reinterpret_cast<const half8_t*>(
                    &sB[buf][(wn + j * 32 + lrow) * kLdsRow + kk * 16 + lk]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0,
                                                                       0, 0);
        }
        if (ks + 1 < ksteps) sstore(buf ^ 1);
        __syncthreads();
    }

    // D layout of a 32x32 MFMA: lane holds column (lane & 31); accumulator e holds
    // row 8*(e/4) + 4*(lane/32) + (e%4).
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int n = n0 + wn + j * 32 + (lane & 31);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + wm + i * 32 + 8 * (e / 4) + 4 * (lane >> 5) + (e % 4);
                if (m < M && n < N) Y[(size_t)m * N + n] = (half_t)acc[i][j][e];
            }
        }
}

template <int BM, int BN, int BS>
static int launch_gemm4(const half_t* A, const uint8_t* B, const half_t* S, const uint8_t* Z,
                        half_t* Y, int M, int N, int K, int nb, hipStream_t st) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    hipLaunchKernelGGL((mnb_gemm4_kernel<BM, BN, BS>), dim3(tiles_m * tiles_n), dim3(256), 0, st,
                       A, B, S, Z, Y, M, N, K, nb, tiles_m, tiles_n);
    return check_launch("mnb_gemm4");
}

template <int BS>
static int dispatch_gemm4(const half_t* A, const uint8_t* B, const half_t* S, const uint8_t* Z,
                          half_t* Y, int M, int N, int K, int nb, hipStream_t st) {
    const long big = (long)((M + 127) / 128) * ((N + 127) / 128);
    if (big >= 2L * device_cu_count()) return launch_gemm4<128, 128, BS>(A, B, S, Z, Y, M, N, K, nb, st);
    return launch_gemm4<64, 128, BS>(A, B, S, Z, Y, M, N, K, nb, st);
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
    if (fast_form && M == 1 && (size_t)nb * bs * sizeof(float) <= 64 * 1024) {
        int rc = -1;
        if (bs == 32) rc = launch_gemv4<T, 32>(a, B, s, Z, y, N, K, nb, st);
        if (bs == 64) rc = launch_gemv4<T, 64>(a, B, s, Z, y, N, K, nb, st);
        if (bs == 128) rc = launch_gemv4<T, 128>(a, B, s, Z, y, N, K, nb, st);
        if (rc >= 0) return rc;
    }
    if constexpr (sizeof(T) == 2 && !std::is_same<T, uint16_t>::value) {
        const bool a_aligned = (reinterpret_cast<uintptr_t>(A) % 16) == 0 && K % 8 == 0;
        if (fast_form && M > 1 && a_aligned) {
            if (bs == 32) return dispatch_gemm4<32>(a, B, s, Z, y, M, N, K, nb, st);
            if (bs == 64) return dispatch_gemm4<64>(a, B, s, Z, y, M, N, K, nb, st);
            if (bs == 128) return dispatch_gemm4<128>(a, B, s, Z, y, M, N, K, nb, st);
        }
    }
    return launch_generic<T>(a, B, s, Z, y, M, N, K, nb, bits, bs, st);
}

}  // namespace ortmi

using namespace ortmi;

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
