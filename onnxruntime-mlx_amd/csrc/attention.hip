// GroupQueryAttention, PagedAttention and RotaryEmbedding for gfx950.
//
// Kernels:
//  * gqa_prep / paged_prep - per new token: optional QK RMS-norm, RoPE on Q and K
//    (fp32 math, one rounding to the op dtype), new K/V written to their cache
//    rows (dense present buffer or paged slot); rotated Q (and, paged, rotated K)
//    staged in the workspace. paged_prep also builds the tile map on the device
//    and clears the per-row split counts.
//  * gqa_decode - S == 1 over a dense [B,KV,T,hd] cache. One workgroup per
//    (batch, kv head, key split); it reads each K/V row once for all H/KV query
//    heads of the group (16 lanes x 16 bytes per 128-dim row, a wave covers 4
//    contiguous rows per load), and in the growing contract writes the same rows
//    to `present` from the registers it already holds, so the past->present copy
//    costs no extra read. Partial softmax states are merged by attn_merge.
//  * gqa_tile / paged_tile - matrix-core flash-attention tiles for everything
//    with more than one query token (GQA prefill, PagedAttention prefill
//    chunks): S^T = K.Q^T and O^T += V^T.P^T on v_mfma_f32_32x32x16_f16, Q^T
//    and K staged in LDS, V transposed in LDS, online softmax in fp32 with one
//    query per lane. Paged keys are fetched through the block table on the
//    device; no control tensor is read back to the host.
//  * paged_decode - one-token PagedAttention rows on the vector units, split-K.
//  * attn_merge / paged_merge - log-sum-exp merge of split-K partials.
#include <mutex>
#include <type_traits>

#include "common.h"

namespace ortmi {

// ------------------------------------------------------------------ RoPE --

// Rotate dims [off, off + 2*half) of a head vector held in `v` (fp32), in place.
// Non-interleaved pairs (i, i+half) and interleaved pairs (2i, 2i+1) follow
// rust/src/ops/attention.rs:1234-1282.
template <typename T>
__device__ __forceinline__ void rope_pair_index(int i, int half, int interleaved, int& ia,
                                                int& ib) {
    if (interleaved) {
        ia = 2 * i;
        ib = 2 * i + 1;
    } else {
        ia = i;
        ib = i + half;
    }
}

// One wave per head vector: lane l handles pairs l, l + 64, ... The wave's own LDS
// accesses stay in program order, so no barrier is needed between its steps.
template <typename T>
__device__ void rope_head_lds(float* v, const T* cos_row, const T* sin_row, int half,
                              int interleaved, int off) {
    for (int i = threadIdx.x & 63; i < half; i += 64) {
        int ia, ib;
        rope_pair_index<T>(i, half, interleaved, ia, ib);
        const float c = to_f32(cos_row[i]), s = to_f32(sin_row[i]);
        const float a = v[off + ia], b = v[off + ib];
        v[off + ia] = a * c - b * s;
        v[off + ib] = b * c + a * s;
    }
}

// RMS-normalise a head vector in LDS (one wave per vector), scale by w.
template <typename T>
__device__ void rms_head_lds(float* v, int hd, const T* w, float eps) {
    const int lane = threadIdx.x & 63;
    float ss = 0.f;
    for (int d = lane; d < hd; d += 64) ss += v[d] * v[d];
    const float inv = 1.0f / sqrtf(wave_sum(ss) / hd + eps);
    for (int d = lane; d < hd; d += 64) v[d] = round_to<T>(v[d] * inv * to_f32(w[d]));
}

// Heads per prep workgroup, one wave each (fewer, fuller workgroups).
constexpr int kPrepHeads = 4;

// 16-bit element <-> its storage bits (fp32 rows never take the pair path).
template <typename T>
__device__ __forceinline__ T bits16_to(uint16_t b) {
    if constexpr (sizeof(T) == 2) return __builtin_bit_cast(T, b);
    else return T(0);
}
template <typename T>
__device__ __forceinline__ uint32_t to_bits16(T x) {
    if constexpr (sizeof(T) == 2) return __builtin_bit_cast(uint16_t, x);
    else return 0u;
}
// Row traffic of the prep kernels in element pairs, one 32-bit access each (a
// 128-dim row is one load instruction per wave instead of two 16-bit ones per
// lane); a row start that is not 4-byte aligned, or a 32-bit row, takes single
// elements.
template <typename T>
__device__ __forceinline__ bool pair_aligned(const T* p) {
    return (reinterpret_cast<uintptr_t>(p) & 3) == 0;
}
template <typename T>
__device__ __forceinline__ void row_to_lds(float* sv, const T* src, int hd, int lane) {
    if (sizeof(T) == 2 && pair_aligned(src)) {
        for (int d2 = lane; d2 < hd / 2; d2 += 64) {
            const uint32_t w = reinterpret_cast<const uint32_t*>(src)[d2];
            sv[2 * d2] = to_f32(bits16_to<T>((uint16_t)(w & 0xffffu)));
            sv[2 * d2 + 1] = to_f32(bits16_to<T>((uint16_t)(w >> 16)));
        }
    } else {
        for (int d = lane; d < hd; d += 64) sv[d] = to_f32(src[d]);
    }
}
template <typename T>
__device__ __forceinline__ void lds_to_row(T* dst, const float* sv, int hd, int lane) {
    if (sizeof(T) == 2 && pair_aligned(dst)) {
        for (int d2 = lane; d2 < hd / 2; d2 += 64) {
            const uint32_t lo = to_bits16(from_f32<T>(sv[2 * d2]));
            const uint32_t hi = to_bits16(from_f32<T>(sv[2 * d2 + 1]));
            reinterpret_cast<uint32_t*>(dst)[d2] = lo | (hi << 16);
        }
    } else {
        for (int d = lane; d < hd; d += 64) dst[d] = from_f32<T>(sv[d]);
    }
}
template <typename T>
__device__ __forceinline__ void copy_row(T* dst, const T* src, int n, int lane) {
    if (sizeof(T) == 2 && pair_aligned(dst) && pair_aligned(src)) {
        for (int d2 = lane; d2 < n / 2; d2 += 64)
            reinterpret_cast<uint32_t*>(dst)[d2] = reinterpret_cast<const uint32_t*>(src)[d2];
    } else {
        for (int d = lane; d < n; d += 64) dst[d] = src[d];
    }
}

// -------------------------------------------------------------- GQA prep --

// One wave per (token, head), kPrepHeads heads per workgroup, with heads
// 0..H-1 = query, H..H+KV-1 = key. Rotated Q goes to qrot [B*S, H, hd]; rotated K
// and raw V go to present rows valid_past + s.
template <typename T>
__global__ __launch_bounds__(64 * kPrepHeads) void gqa_prep_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ cos_c, const T* __restrict__ sin_c, int half, int interleaved,
    T* __restrict__ qrot, T* __restrict__ pk, T* __restrict__ pv, int B, int S, int H, int KV,
    int hd, int64_t pcap, int vp, int64_t q_stride, int64_t kv_stride) {
    extern __shared__ float sv_all[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tok = blockIdx.x;  // b*S + s
    const int head = blockIdx.y * kPrepHeads + wave;
    if (head >= H + KV) return;
    float* sv = sv_all + wave * hd;
    const int b = tok / S, s = tok % S;
    const int pos = vp + s;
    const bool is_q = head < H;
    const T* src = is_q ? q + (int64_t)tok * q_stride + (int64_t)head * hd
                        : k + (int64_t)tok * kv_stride + (int64_t)(head - H) * hd;
    row_to_lds<T>(sv, src, hd, lane);
    if (cos_c) rope_head_lds<T>(sv, cos_c + (int64_t)pos * half, sin_c + (int64_t)pos * half, half,
                                interleaved, 0);
    if (is_q) {
        lds_to_row<T>(qrot + ((int64_t)tok * H + head) * hd, sv, hd, lane);
    } else {
        const int kvh = head - H;
        const int64_t row = (((int64_t)b * KV + kvh) * pcap + pos) * hd;
        lds_to_row<T>(pk + row, sv, hd, lane);
        copy_row<T>(pv + row, v + (int64_t)tok * kv_stride + (int64_t)kvh * hd, hd, lane);
    }
}

__global__ __launch_bounds__(256) void kv_copy_kernel(const uint4* __restrict__ src,
                                                      uint4* __restrict__ dst, int64_t src_cap,
                                                      int64_t dst_cap, int64_t copy_rows,
                                                      int vec_per_row, int64_t total_vec) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total_vec; i += stride) {
        const int64_t per_head = copy_rows * vec_per_row;
        const int64_t bh = i / per_head;
        const int64_t rem = i % per_head;
        dst[bh * dst_cap * vec_per_row + rem] = src[bh * src_cap * vec_per_row + rem];
    }
}

// ---------------------------------------------------------- GQA decode --

// cos/sin entries that rotate this lane's 8 dims, as raw storage bits (widened
// where they are used). Non-interleaved dim d < 2*half uses entry d mod half;
// an interleaved pair (2p, 2p+1) uses entry p, kept at index 2p - dl. Entries the
// lane does not use read as zero without a memory access (offset past the row),
// so the loads are unconditional. `half` == 0 loads nothing.
struct RopeLane {
    uint32_t c[8], s[8];
};
template <typename T>
__device__ __forceinline__ uint32_t load_elem_bits(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    if constexpr (sizeof(T) == 4)
        return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    else
        return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
template <typename T>
__device__ __forceinline__ float elem_from_bits(uint32_t v) {
    if constexpr (std::is_same<T, float>::value)
        return __uint_as_float(v);
    else if constexpr (std::is_same<T, half_t>::value)
        return (float)__builtin_bit_cast(half_t, (uint16_t)v);
    else
        return to_f32((uint16_t)v);  // bf16 bits
}
template <typename T>
__device__ __forceinline__ RopeLane rope_fetch(const T* c, const T* s, int half, int dl,
                                               int interleaved) {
    const uint32_t bytes = (uint32_t)half * sizeof(T);
    const __amdgpu_buffer_rsrc_t rc = buffer_rsrc(c, bytes), rs = buffer_rsrc(s, bytes);
    RopeLane r;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int d = dl + i;
        int p = d < half ? d : d - half;
        bool use = d < 2 * half;
        if (interleaved) {
            p = d / 2;
            use = (i % 2 == 0) && d + 1 < 2 * half;
        }
        const uint32_t off = use ? (uint32_t)p * sizeof(T) : bytes;
        r.c[i] = load_elem_bits<T>(rc, off);
        r.s[i] = load_elem_bits<T>(rs, off);
    }
    return r;
}
// Rotate the 8 dims [dl, dl+8) held by this lane (head vector spread over LPR
// lanes, 8 dims each) with table entries from rope_fetch. Non-interleaved pairs
// (i, i+half) live `half/8` lanes apart and are exchanged with a shuffle;
// interleaved pairs sit inside the lane.
template <typename T, int LPR>
__device__ __forceinline__ void rope_apply(float (&x)[8], int dl, const RopeLane& r, int half,
                                           int interleaved) {
    if (interleaved) {
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            if (dl + i + 1 < 2 * half) {
                const float cs = elem_from_bits<T>(r.c[i]), sn = elem_from_bits<T>(r.s[i]);
                const float a = x[i], b = x[i + 1];
                x[i] = a * cs - b * sn;
                x[i + 1] = b * cs + a * sn;
            }
        }
        return;
    }
    const int off = half / 8;
    const int lane = threadIdx.x & 63;
    float partner[8];
    const bool lowhalf = dl < half;
    const int src = lowhalf ? lane + off : lane - off;
    if (LPR == 16 && off == 8) {
#pragma unroll
        for (int i = 0; i < 8; ++i) partner[i] = dpp_mov<0x128>(x[i]);  // row_ror:8
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) partner[i] = __shfl(x[i], src, 64);
    }
    if (dl < 2 * half) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float cs = elem_from_bits<T>(r.c[i]), sn = elem_from_bits<T>(r.s[i]);
            x[i] = lowhalf ? x[i] * cs - partner[i] * sn : x[i] * cs + partner[i] * sn;
        }
    }
}

// End of a decode workgroup (NW waves, lane groups of LPR lanes each holding an
// online-softmax state (m, l, o[8] over dims dl..dl+7) for G heads): merges the
// groups of each wave with cross-lane reductions, then the NW waves through LDS,
// and calls emit(g, d, M, L, acc) once per (head, dim) with the merged state.
template <int HD, int G, int LPR, int NW, typename Emit>
__device__ __forceinline__ void decode_merge(float (&m)[G], float (&l)[G], float (&o)[G][8],
                                             float (&s_m)[NW][G], float (&s_l)[NW][G],
                                             float (&s_o)[NW][G][HD], Emit emit) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int dl = (lane % LPR) * 8;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        float mw = m[g];
        if constexpr (LPR == 8) mw = fmaxf(mw, dpp_mov<0x128>(mw));
        if constexpr (LPR <= 16) {
            const LanePair p = swap16(mw);
            mw = fmaxf(p.a, p.b);
        }
        const LanePair p = swap32(mw);
        mw = fmaxf(p.a, p.b);
        const float f = m[g] == -INFINITY ? 0.f : __expf(m[g] - mw);
        l[g] = across_groups_sum<LPR>(l[g] * f);
        m[g] = mw;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = across_groups_sum<LPR>(o[g][i] * f);
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            s_m[wave][g] = m[g];
            s_l[wave][g] = l[g];
        }
    }
    if (lane < LPR) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int i = 0; i < 8; ++i) s_o[wave][g][dl + i] = o[g][i];
    }
    __syncthreads();
    for (int idx = tid; idx < G * HD; idx += 64 * NW) {
        const int g = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, s_m[w][g]);
        float L = 0.f, acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float mw = s_m[w][g];
            const float f = mw == -INFINITY ? 0.f : __expf(mw - M);
            L += s_l[w][g] * f;
            acc += s_o[w][g][d] * f;
        }
        emit(g, d, M, L, acc);
    }
}

// Each lane group of LPR lanes owns one row per step; scores use a blocked
// online softmax. In the growing contract rows below vp are copied from past to
// present out of the registers already loaded. Head 96 runs on 16-lane groups
// like head 128: its last 4 lanes of each group are padding that loads and
// stores nothing and adds zeros.
template <typename T, int HD, int G>
__global__ __launch_bounds__(256) void gqa_decode_kernel(
    const T* __restrict__ q, const T* __restrict__ knew, const T* __restrict__ vnew,
    int64_t q_stride, int64_t kv_stride, const T* __restrict__ cos_c, const T* __restrict__ sin_c,
    int half, int interleaved, const T* __restrict__ kpast, const T* __restrict__ vpast,
    T* __restrict__ kpres, T* __restrict__ vpres, int64_t past_cap, int64_t pres_cap,
    int copy_past, int vp, int chunk, int nsplit, int KV, float scale, float* __restrict__ part,
    T* __restrict__ out, const int* __restrict__ total_dev, int vp_max, int gsplit) {
    static_assert(HD == 64 || HD == 96 || HD == 128, "head size");
    constexpr int LPR = HD <= 64 ? 8 : 16;  // lanes per row (16 bytes each; head 96 padded)
    constexpr int HDP = 8 * LPR;            // head dims the lane groups span
    constexpr int RPW = 64 / LPR;        // rows per wave per step
    constexpr int NW = 4;                // waves
    constexpr int RPS = NW * RPW;        // rows per workgroup step
    constexpr int U = G <= 4 ? 4 : 2;    // steps per online-softmax block (registers)
    constexpr int BLK = RPS * U;         // rows per block
    __shared__ float s_o[NW][G][HDP];
    __shared__ float s_m[NW][G], s_l[NW][G];

    // blockIdx.x = (b*KV + kvh) * gsplit + head group: the G*gsplit query heads of
    // a KV head may be spread over gsplit workgroups that read the same rows.
    const int bk = blockIdx.x / gsplit;
    const int hgrp = blockIdx.x % gsplit;
    const int split = blockIdx.y;
    const int b = bk / KV, kvh = bk % KV;
    const int GT = G * gsplit;  // query heads per KV head
    const int H = KV * GT;
    const int h0 = kvh * GT + hgrp * G;  // first query head of this workgroup
    const int j0 = split * chunk;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / LPR;
    const int dl = (lane % LPR) * 8;
    const bool padl = dl >= HD;  // a padding lane of head 96
    T* kw = kpres + (int64_t)bk * pres_cap * HD;
    T* vw = vpres + (int64_t)bk * pres_cap * HD;
    const T* kbase = copy_past ? kpast + (int64_t)bk * past_cap * HD : kw;
    const T* vbase = copy_past ? vpast + (int64_t)bk * past_cap * HD : vw;
    const int64_t src_rows = copy_past ? past_cap : pres_cap;

    // Every global access below is unconditional (a branch around a load makes the
    // compiler wait for every load in flight where the paths join, which would
    // drain the block prefetch). Rows of this (b, kv) slice go through raw buffer
    // accesses: a row outside the split, or a store that must not happen, gets an
    // offset past the slice and touches no memory.
    const uint32_t row_bytes = HD * sizeof(T);
    const uint32_t src_end = (uint32_t)src_rows * row_bytes;
    const uint32_t pres_end = (uint32_t)pres_cap * row_bytes;
    const __amdgpu_buffer_rsrc_t rsk = buffer_rsrc(kbase, src_end);
    const __amdgpu_buffer_rsrc_t rsv = buffer_rsrc(vbase, src_end);
    const __amdgpu_buffer_rsrc_t rdk = buffer_rsrc(kw, pres_end);
    const __amdgpu_buffer_rsrc_t rdv = buffer_rsrc(vw, pres_end);
    const uint32_t lane_off = (uint32_t)(dl * sizeof(T));

    // 1. Loads independent of the past length, then the first block of rows.
    // (A scalar load: its wait does not count vector memory operations.)
    int tv = 0;
    if (total_dev) tv = total_dev[0];
    // Padding lanes read the head's first 8 dims (in bounds) and zero them.
    const int dlr = padl ? 0 : dl;
    const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
    uint4 qraw[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const uint4 v = *reinterpret_cast<const uint4*>(q + (int64_t)b * q_stride +
                                                        (int64_t)(h0 + g) * HD + dlr);
        qraw[g] = padl ? zero4 : v;
    }
    const uint4 kraw0 = *reinterpret_cast<const uint4*>(knew + (int64_t)b * kv_stride +
                                                        (int64_t)kvh * HD + dlr);
    const uint4 vraw0 = *reinterpret_cast<const uint4*>(vnew + (int64_t)b * kv_stride +
                                                        (int64_t)kvh * HD + dlr);
    const uint4 kraw = padl ? zero4 : kraw0;
    const uint4 vraw = padl ? zero4 : vraw0;
    // Rows [base, base + BLK) below `lim`; rows at or past src_rows fall outside
    // the slice and read zeros. Rows are streamed once per step: loads and the
    // copy stores are non-temporal (measured 5% faster on the 4096-row copy).
    auto load_block = [&](u32x4_t (&kk)[U], u32x4_t (&vv)[U], int base, int lim) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = base + u * RPS + wave * RPW + sub;
            const uint32_t off =
                j < lim && j < src_rows && !padl ? (uint32_t)j * row_bytes + lane_off : src_end;
            kk[u] = __builtin_amdgcn_raw_buffer_load_b128(rsk, off, 0, kCachePolicyNT);
            vv[u] = __builtin_amdgcn_raw_buffer_load_b128(rsv, off, 0, kCachePolicyNT);
        }
    };
    // Three register sets in rotation. A set is reloaded only after another
    // block's loads were issued behind its copy stores, so waiting for those
    // stores (the counter retires in order) never waits for a block still ahead.
    u32x4_t ka[U], va[U], kb[U], vb[U], kc[U], vc[U];
    load_block(ka, va, j0, j0 + chunk);

    // 2. Past length, the rotary table entries, the second block.
    if (total_dev) vp = min(max(tv - 1, 0), vp_max);
    // The last split runs to the end: splits are sized over the cached rows, and
    // the new row (and any rows past nsplit * chunk) fall to it.
    const int nkeys = vp + 1;
    const int j1 = split == nsplit - 1 ? nkeys : min(nkeys, j0 + chunk);
    const bool rot = cos_c != nullptr;
    const RopeLane rl = rope_fetch<T>(rot ? cos_c + (int64_t)vp * half : q,
                                      rot ? sin_c + (int64_t)vp * half : q, rot ? half : 0, dl,
                                      interleaved);
    load_block(kb, vb, j0 + BLK, j1);

    // 3. RoPE of the queries and of the new key. Scores are kept as raw dot
    // products of the rounded query with the keys; the softmax scale (and log2 e,
    // for the hardware exp2) is applied inside the exponent.
    constexpr bool kDot2 = std::is_same<T, half_t>::value;
    float qf[G][8];
    half2_t q2[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const T* rv = reinterpret_cast<const T*>(&qraw[g]);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[g][i] = to_f32(rv[i]);
        if (rot) rope_apply<T, LPR>(qf[g], dl, rl, half, interleaved);
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[g][i] = round_to<T>(qf[g][i]);
#pragma unroll
        for (int p = 0; p < 4; ++p) q2[g][p] = half2_t{(half_t)qf[g][2 * p], (half_t)qf[g][2 * p + 1]};
    }
    float knf[8], vnf[8];
    {
        const T* rk = reinterpret_cast<const T*>(&kraw);
        const T* rvv = reinterpret_cast<const T*>(&vraw);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            knf[i] = to_f32(rk[i]);
            vnf[i] = to_f32(rvv[i]);
        }
        if (rot) rope_apply<T, LPR>(knf, dl, rl, half, interleaved);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            knf[i] = round_to<T>(knf[i]);  // the stored (rounded) key is what gets attended
    }
    // The new key's storage bits (stored to row vp and attended like a cache row).
    u32x4_t knb;
    {
        T kt[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kt[i] = from_f32<T>(knf[i]);
        __builtin_memcpy(&knb, kt, sizeof(knb));
    }
    constexpr float kLog2e = 1.4426950408889634f;
    const float c2 = scale * kLog2e;
    // Partial dot product of a head's query with 8 dims of a key (this lane's).
    auto qk = [&](int g, const u32x4_t& kv) -> float {
        float d = 0.f;
        if constexpr (kDot2) {
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint32_t w = kv[p];  // (a bit_cast of kv[p] itself reads element 0)
                d = __builtin_amdgcn_fdot2(q2[g][p], __builtin_bit_cast(half2_t, w), d, false);
            }
        } else {
            const T* kt = reinterpret_cast<const T*>(&kv);
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(qf[g][i], to_f32(kt[i]), d);
        }
        return d;
    };

    float m[G], l[G], o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
    }
    // Online-softmax update with a block's raw scores (masked rows at -inf);
    // `vrow(u, i)` gives the value of row u, dim i.
    auto absorb = [&](float (&sc)[U][G], auto vrow) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float bmax = sc[0][g];
#pragma unroll
            for (int u = 1; u < U; ++u) bmax = fmaxf(bmax, sc[u][g]);
            const float mn = fmaxf(m[g], bmax);
            // m = -inf (nothing seen yet) gives alpha 0; mn = -inf keeps everything 0.
            const float alpha =
                m[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m[g] - mn) * c2);
            l[g] *= alpha;
#pragma unroll
            for (int i = 0; i < 8; ++i) o[g][i] *= alpha;
            m[g] = mn;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float vf[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) vf[i] = vrow(u, i);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = sc[u][g] == -INFINITY
                                    ? 0.f
                                    : __builtin_amdgcn_exp2f(fmaf(sc[u][g], c2, -m[g] * c2));
                l[g] += p;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[g][i] = fmaf(p, vf[i], o[g][i]);
            }
        }
    };
    // Rows of the walk: [j0, jw); the new row vp (if this split owns it) is
    // attended separately from registers.
    const bool own_new = vp >= j0 && vp < j1;
    const int jw = own_new ? vp : j1;
    const bool copier = copy_past && hgrp == 0;
    auto process = [&](const u32x4_t (&kk)[U], const u32x4_t (&vv)[U], int base) {
        float sc[U][G];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = base + u * RPS + wave * RPW + sub;
            // Past rows below vp are copied into the present buffer.
            const uint32_t coff =
                copier && j < jw && !padl ? (uint32_t)j * row_bytes + lane_off : pres_end;
            __builtin_amdgcn_raw_buffer_store_b128(kk[u], rdk, coff, 0, kCachePolicyNT);
            __builtin_amdgcn_raw_buffer_store_b128(vv[u], rdv, coff, 0, kCachePolicyNT);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float d = group_sum<LPR>(qk(g, kk[u]));
                sc[u][g] = j < jw ? d : -INFINITY;
            }
        }
        absorb(sc, [&](int u, int i) { return to_f32(reinterpret_cast<const T*>(&vv[u])[i]); });
    };
    // 4. Blocks, two ahead of the one being processed. Loads past j1 touch no memory.
    for (int base = j0; base < jw; base += 3 * BLK) {
        process(ka, va, base);
        load_block(kc, vc, base + 2 * BLK, jw);
        if (base + BLK >= jw) break;
        process(kb, vb, base + BLK);
        load_block(ka, va, base + 3 * BLK, jw);
        if (base + 2 * BLK >= jw) break;
        process(kc, vc, base + 2 * BLK);
        load_block(kb, vb, base + 4 * BLK, jw);
    }
    if (own_new) {
        // One lane group (wave 0, sub-row 0) takes the new row; the others see it
        // masked, so it is counted once when the groups are merged.
        float sc[U][G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float d = group_sum<LPR>(qk(g, knb));
#pragma unroll
            for (int u = 0; u < U; ++u) sc[u][g] = u == 0 && wave == 0 && sub == 0 ? d : -INFINITY;
        }
        absorb(sc, [&](int, int i) { return vnf[i]; });
    }
    // Back to natural-log units for the merges (scores times the scale).
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (m[g] != -INFINITY) m[g] *= scale;
    // The new row (RoPE'd key, value) goes to row vp of the present buffer, from
    // the split that owns it; it is written last so no reload waits on it.
    {
        const uint32_t noff = own_new && hgrp == 0 && wave == 0 && sub == 0 && !padl
                                  ? (uint32_t)vp * row_bytes + lane_off
                                  : pres_end;
        __builtin_amdgcn_raw_buffer_store_b128(knb, rdk, noff, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{vraw.x, vraw.y, vraw.z, vraw.w}, rdv,
                                               noff, 0, 0);
    }
    // out == null: split partials only (even for one split), merged by the consumer.
    decode_merge<HDP, G, LPR, NW>(m, l, o, s_m, s_l, s_o, [&](int g, int d, float M, float L, float acc) {
        if (d >= HD) return;  // padding dims of head 96
        const int64_t row = (int64_t)b * H + h0 + g;
        if (nsplit == 1 && out) {
            out[row * HD + d] = from_f32<T>(L > 0.f ? acc / L : 0.f);
            return;
        }
        float* dst = part + (row * nsplit + split) * (HD + 2);
        dst[d] = acc;
        if (d == 0) {
            dst[HD] = M;
            dst[HD + 1] = L;
        }
    });
}

// Merge split partials: out[row][d] = sum_i o_i e^{m_i-M} / sum_i l_i e^{m_i-M}.
// One workgroup per row. Up to kMergeFast splits with vhd <= 128 (one dim per
// thread), every value a thread needs is requested in one batch of loads (splits
// past the count read zeros without an access) and merged in registers. Larger
// cases compute the split weights once into LDS, then each thread sums its
// output dims over the splits.
constexpr int kMergeFast = 16;
// Most key splits of a dense prefill tile (each split writes a partial row).
constexpr int kPrefillSplits = 2;
template <typename T>
__global__ __launch_bounds__(128) void attn_merge_kernel(const float* __restrict__ part,
                                                         T* __restrict__ out, int nsplit,
                                                         const int* __restrict__ nsplit_row,
                                                         int vhd, int H,
                                                         int64_t out_tok_stride,
                                                         const int* __restrict__ row_map) {
    __shared__ float s_w[1024];
    __shared__ float s_red[2];
    const int r = blockIdx.x;
    int orow = r;
    if (row_map) {
        orow = row_map[r];
        if (orow < 0) return;
    }
    const int ns = min(1024, nsplit_row ? nsplit_row[r] : nsplit);
    const float* p = part + (int64_t)r * nsplit * (vhd + 2);
    if (ns <= kMergeFast && vhd <= 128) {
        const uint32_t bytes = (uint32_t)(ns * (vhd + 2)) * 4u;
        const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(p, bytes);
        const int d = min((int)threadIdx.x, vhd - 1);
        float mv[kMergeFast], lv[kMergeFast], ov[kMergeFast];
#pragma unroll
        for (int i = 0; i < kMergeFast; ++i) {
            const uint32_t row = (uint32_t)(i * (vhd + 2)) * 4u;
            const bool in = i < ns;
            mv[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rp, in ? row + vhd * 4u : bytes, 0, 0));
            lv[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rp, in ? row + vhd * 4u + 4u : bytes, 0, 0));
            ov[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rp, in ? row + d * 4u : bytes, 0, 0));
        }
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < kMergeFast; ++i)
            if (i < ns) M = fmaxf(M, mv[i]);
        float L = 0.f, acc = 0.f;
#pragma unroll
        for (int i = 0; i < kMergeFast; ++i) {
            const float w = i < ns && mv[i] != -INFINITY ? __expf(mv[i] - M) : 0.f;
            L = fmaf(w, lv[i], L);
            acc = fmaf(w, ov[i], acc);
        }
        if ((int)threadIdx.x < vhd) {
            T* o = out + (int64_t)(orow / H) * out_tok_stride + (int64_t)(orow % H) * vhd;
            o[threadIdx.x] = from_f32<T>(L > 0.f ? acc / L : 0.f);
        }
        return;
    }
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < ns; i += blockDim.x) mx = fmaxf(mx, p[i * (vhd + 2) + vhd]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = mx;
    __syncthreads();
    const float M = fmaxf(s_red[0], s_red[1]);
    __syncthreads();
    float lsum = 0.f;
    for (int i = threadIdx.x; i < ns; i += blockDim.x) {
        const float m = p[i * (vhd + 2) + vhd];
        const float w = m == -INFINITY ? 0.f : __expf(m - M);
        s_w[i] = w;
        lsum += w * p[i * (vhd + 2) + vhd + 1];
    }
    lsum = wave_sum(lsum);
    if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = lsum;
    __syncthreads();
    const float L = s_red[0] + s_red[1];
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    T* o = out + (int64_t)(orow / H) * out_tok_stride + (int64_t)(orow % H) * vhd;
    for (int d = threadIdx.x; d < vhd; d += blockDim.x) {
        float acc = 0.f;
#pragma unroll 8
        for (int i = 0; i < ns; ++i) acc = fmaf(p[i * (vhd + 2) + d], s_w[i], acc);
        o[d] = from_f32<T>(acc * inv);
    }
}

// ------------------------------------------------------------ attn_tile --

// Key/value source for one (sequence, kv head).
struct DenseKV {
    // [B, KV, cap, hd]
    const void* k;
    const void* v;
    int64_t cap;
    int KV;
};
struct PagedKV {
    const void* kcache;  // [nblk, blk, KV, hd]
    const void* vcache;  // [nblk, blk, KV, vhd] or null (latent)
    const void* knew;    // rotated new keys [T, KV, hd]
    const void* vnew;    // raw new values [T, KV*vhd] or null (latent)
    const int32_t* bt;
    int64_t nblk;
    int blk, maxb, KV;
    int blk_shift;  // log2(blk) when blk is a power of two, else -1
    int max_ctx;    // keys at positions >= max_ctx are not attended
};

struct TileDesc {
    int seq;        // sequence index
    int tok0;       // first token (packed row) of the tile
    int ntok;       // tokens in the tile
    int qpos0;      // absolute position of the first query token
    int past;       // keys [0, past) come from the cache
    int nkeys;      // total keys (past + new tokens of the sequence)
    int tok_seq0;   // first packed token of the sequence (paged)
};

constexpr int kTileRows = 64;   // max query rows per workgroup
constexpr int kKeyTile = 64;

template <typename T, int HD, int VHD, bool PAGED>
__device__ __forceinline__ const T* key_ptr(const DenseKV& d, const PagedKV& p, const TileDesc& t,
                                            int b, int kvh, int j, bool value) {
    if constexpr (!PAGED) {
        const T* base = static_cast<const T*>(value ? d.v : d.k);
        return base + (((int64_t)b * d.KV + kvh) * d.cap + j) * (value ? VHD : HD);
    } else {
        if (j >= t.past) {
            const int tok = t.tok_seq0 + (j - t.past);
            if (value && p.vnew)
                return static_cast<const T*>(p.vnew) + ((int64_t)tok * p.KV + kvh) * VHD;
            return static_cast<const T*>(p.knew) + ((int64_t)tok * p.KV + kvh) * HD;
        }
        const int lb = j / p.blk;
        const int phys = (j >= 0 && lb < p.maxb) ? p.bt[(int64_t)t.seq * p.maxb + lb] : -1;
        if (phys < 0 || phys >= p.nblk) return nullptr;
        const int64_t slot = (int64_t)phys * p.blk + (j % p.blk);
        if (value && p.vcache)
            return static_cast<const T*>(p.vcache) + (slot * p.KV + kvh) * VHD;
        return static_cast<const T*>(p.kcache) + (slot * p.KV + kvh) * HD;
    }
}

// One workgroup: `rows` = ntok * G query rows (row r -> token r / G, head r % G
// of the group) against keys [k0, k1) of one (sequence, kv head). When
// `part` is null the normalised output is written; otherwise the partial state.
template <typename T, int HD, int VHD, bool PAGED>
__device__ void attn_tile_body(const TileDesc& t, int kvh, int G, int H, const T* __restrict__ qrot,
                               const DenseKV& dk, const PagedKV& pk, float scale,
                               const float* __restrict__ sink, int k0, int k1,
                               T* __restrict__ out, int64_t out_tok_stride,
                               float* __restrict__ part, int nsplit, int split) {
    __shared__ float sQ[kTileRows][HD + 1];
    __shared__ T sK[kKeyTile][HD + 8];
    __shared__ T sV[kKeyTile][VHD + 8];
    __shared__ float sS[kTileRows][kKeyTile + 1];
    __shared__ float sM[kTileRows], sL[kTileRows], sAlpha[kTileRows];
    __shared__ int sOk[kKeyTile];

    const int tid = threadIdx.x;
    const int rows = t.ntok * G;
    for (int idx = tid; idx < kTileRows * HD; idx += 256) {
        const int r = idx / HD, d = idx % HD;
        float v = 0.f;
        if (r < rows) {
            const int tok = t.tok0 + r / G, h = kvh * G + r % G;
            v = to_f32(qrot[((int64_t)tok * H + h) * HD + d]) * scale;
        }
        sQ[r][d] = v;
    }
    if (tid < kTileRows) {
        sM[tid] = -INFINITY;
        sL[tid] = 0.f;
    }
    // Thread -> (row, 16-key slice) for scores; (row, VHD/4 dims) for P.V.
    const int r_s = tid / 4, c_s = (tid % 4) * 16;
    constexpr int DV = VHD / 4;
    const int d_o = (tid % 4) * DV;
    float o[DV];
#pragma unroll
    for (int i = 0; i < DV; ++i) o[i] = 0.f;
    const bool row_live = r_s < rows;
    const int qpos = t.qpos0 + r_s / G;
    __syncthreads();

    for (int kb = k0; kb < k1; kb += kKeyTile) {
        const int nk = min(kKeyTile, k1 - kb);
        // Stage K/V tile (16-byte vectors).
        constexpr int KV_VEC = HD / 8, VV_VEC = VHD / 8;
        for (int idx = tid; idx < kKeyTile * KV_VEC; idx += 256) {
            const int r = idx / KV_VEC, c = (idx % KV_VEC) * 8;
            uint4 val = make_uint4(0, 0, 0, 0);
            const T* p = r < nk ? key_ptr<T, HD, VHD, PAGED>(dk, pk, t, t.seq, kvh, kb + r, false)
                                : nullptr;
            if (p) val = *reinterpret_cast<const uint4*>(p + c);
            *reinterpret_cast<uint4*>(&sK[r][c]) = val;
            if (c == 0) sOk[r] = p != nullptr;
        }
        for (int idx = tid; idx < kKeyTile * VV_VEC; idx += 256) {
            const int r = idx / VV_VEC, c = (idx % VV_VEC) * 8;
            uint4 val = make_uint4(0, 0, 0, 0);
            if (r < nk) {
                const T* p = key_ptr<T, HD, VHD, PAGED>(dk, pk, t, t.seq, kvh, kb + r, true);
                if (p) val = *reinterpret_cast<const uint4*>(p + c);
            }
            *reinterpret_cast<uint4*>(&sV[r][c]) = val;
        }
        __syncthreads();
        // Scores.
        float tmax = -INFINITY;
        if (row_live) {
            for (int c = 0; c < 16; ++c) {
                const int jj = c_s + c, j = kb + jj;
                float sc = -INFINITY;
                const bool ok = jj < nk && j <= qpos && sOk[jj];
                if (ok) {
                    float acc = 0.f;
#pragma unroll 16
                    for (int d = 0; d < HD; ++d) acc = fmaf(sQ[r_s][d], to_f32(sK[jj][d]), acc);
                    sc = acc;
                }
                sS[r_s][jj] = sc;
                tmax = fmaxf(tmax, sc);
            }
        }
        tmax = group_max<4>(tmax);
        __syncthreads();
        if (row_live) {
            const float m_old = sM[r_s];
            const float m_new = fmaxf(m_old, tmax);
            float lsum = 0.f;
            for (int c = 0; c < 16; ++c) {
                const int jj = c_s + c;
                const float e = (m_new == -INFINITY) ? 0.f : __expf(sS[r_s][jj] - m_new);
                sS[r_s][jj] = e;
                lsum += e;
            }
            lsum = group_sum<4>(lsum);  // the 4 lanes of a row share row_live
            const float alpha = (m_old == -INFINITY) ? 0.f : __expf(m_old - m_new);
            if ((tid % 4) == 0) {
                sL[r_s] = sL[r_s] * alpha + lsum;
                sM[r_s] = m_new;
                sAlpha[r_s] = alpha;
            }
        }
        __syncthreads();
        if (row_live) {
            const float alpha = sAlpha[r_s];
#pragma unroll
            for (int i = 0; i < DV; ++i) o[i] *= alpha;
            for (int jj = 0; jj < nk; ++jj) {
                const float p = sS[r_s][jj];
#pragma unroll
                for (int i = 0; i < DV; ++i) o[i] = fmaf(p, to_f32(sV[jj][d_o + i]), o[i]);
            }
        }
        __syncthreads();
    }
    if (!row_live) return;
    const int tok = t.tok0 + r_s / G, h = kvh * G + r_s % G;
    float m = sM[r_s], l = sL[r_s];
    if (part) {
        // Partial rows are token-major: row tok * H + h.
        float* dst = part + (((int64_t)tok * H + h) * nsplit + split) * (VHD + 2);
#pragma unroll
        for (int i = 0; i < DV; ++i) dst[d_o + i] = o[i];
        if ((tid % 4) == 0) {
            dst[VHD] = m;
            dst[VHD + 1] = l;
        }
        return;
    }
    if (sink) {
        const float sv = sink[h];
        const float mm = fmaxf(m, sv);
        const float a = (m == -INFINITY) ? 0.f : __expf(m - mm);
        l = l * a + __expf(sv - mm);
#pragma unroll
        for (int i = 0; i < DV; ++i) o[i] *= a;
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    T* dst = out + (int64_t)tok * out_tok_stride + (int64_t)h * VHD + d_o;
#pragma unroll
    for (int i = 0; i < DV; ++i) dst[i] = from_f32<T>(o[i] * inv);
}

// The attention tile on the matrix cores (fp16), 128 query rows per workgroup,
// computed transposed so that everything a query needs stays in its lanes:
//   S^T = K Q^T     (v_mfma_f32_32x32x16_f16; A = 32 keys x 16 dims from LDS,
//                    B = 16 dims x 32 queries, held in registers for the whole tile)
//   O^T += V^T P^T  (A = 32 head dims x 16 keys from transposed V in LDS,
//                    B = 16 keys x 32 queries = this lane's own probabilities)
// In the accumulator layout a lane holds one query (column lane % 32) and 16 keys
// (or 16 head dims) of it, and the two lanes lane, lane ^ 32 share a query. So the
// online softmax is register arithmetic plus one permlane32 swap per reduction,
// and P never goes through LDS: the k-order of the P V product is permuted to the
// keys a lane already holds (keys {4h..4h+3, 8+4h..8+4h+3} of each 16 for lane half
// h), and V^T is read in that same order. fp32 accumulation; P is rounded to
// fp16 once and the softmax denominator sums the same rounded values.
// Wave w owns queries 32w..32w+31 of the tile. Key blocks of 64 go global ->
// registers -> LDS, the next block's loads in flight while the current one is used.

// 16-bit element pieces of the matrix-core tile: T = half_t (fp16) or uint16_t
// (bf16 bits). Operands travel as 16-bit bit patterns; only the matrix-core step,
// the rounding of P and of the output, and the P row sums depend on the type.
typedef uint16_t u16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
template <typename T>
__device__ __forceinline__ float16_t tile_mfma(u16x8_t a, u16x8_t b, float16_t c) {
    if constexpr (std::is_same<T, half_t>::value)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                      __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                       __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}
// A float rounded to T (round to nearest even), as bits.
template <typename T>
__device__ __forceinline__ uint16_t tile_round(float x) {
    if constexpr (std::is_same<T, half_t>::value)
        return __builtin_bit_cast(uint16_t, (half_t)x);
    else
        return __builtin_bit_cast(uint16_t, (__bf16)x);
}
// Sum of two T values (bits lo, hi of w) added to acc in fp32, exactly widened.
template <typename T>
__device__ __forceinline__ float tile_pair_sum(uint32_t w, float acc) {
    if constexpr (std::is_same<T, half_t>::value) {
        const half2_t one2 = {(half_t)1.f, (half_t)1.f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, w), one2, acc, false);
    } else {
        const bf16x2_t one2 = {(__bf16)1.f, (__bf16)1.f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one2, acc, false);
    }
}

template <typename T, int HD, int VHD, bool PAGED, int NW = 4>
__device__ void attn_mfma_body(const TileDesc& t, int kvh, int G, int H,
                               const T* __restrict__ qrot, const DenseKV& dk,
                               const PagedKV& pk, float scale, const float* __restrict__ sink,
                               int k0, int k1, T* __restrict__ out, int64_t out_tok_stride,
                               float* __restrict__ part, int nsplit, int split) {
    static_assert(std::is_same<T, half_t>::value || std::is_same<T, uint16_t>::value,
                  "fp16 or bf16 (16-bit storage)");
    static_assert(kKeyTile == 64 && HD % 16 == 0 && VHD % 32 == 0, "tile shape");
    static_assert(NW == 4 || NW == 8, "waves per tile");
    constexpr int NT = 64 * NW;       // threads
    constexpr int kRows = 32 * NW;    // query rows of the tile (32 per wave)
    constexpr int KP = HD + 8, VP = kKeyTile + 8;
    constexpr int DT = VHD / 32;          // head-dim tiles of O^T
    __shared__ uint16_t sK[kKeyTile * KP];
    __shared__ uint16_t sVt[VHD * VP];
    __shared__ unsigned long long sOk;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lrow = lane & 31, hh = lane >> 5, lk = hh * 8;
    const int rows = t.ntok * G;
    const int q = wave * 32 + lrow;                // this lane's query row in the tile
    const bool qlive = q < rows;
    const int qpos = t.qpos0 + (qlive ? q / G : 0);
    // Earliest position among the wave's queries: keys up to it are causally
    // visible to every query of the wave.
    const int qpos_wave = t.qpos0 + (wave * 32) / G;
    // Scores are kept in the log2 domain (exp2 is the hardware exponential). The
    // scale is applied inside the exponent, after the block maximum of the raw
    // scores, which needs it positive: a negative scale flips the sign of Q as it
    // is staged (the sign bit, exact in fp16 and bf16) and scales by its magnitude.
    constexpr float kLog2e = 1.4426950408889634f;
    const float sc2 = fabsf(scale) * kLog2e;
    const uint32_t qsign = scale < 0.f ? 0x80008000u : 0u;
    // Q^T operand: the tile's query rows are staged in LDS once (zeros past the
    // last row) and each k-step reads its 8 head dims from there, which keeps
    // HD / 2 VGPRs free for the whole key walk.
    __shared__ uint16_t sQ[kRows * KP];
    {
        constexpr int CPR = HD / 8;  // 16-byte chunks per row
        for (int i = tid; i < kRows * CPR; i += NT) {
            const int r = i / CPR, c = i % CPR;
            u32x4_t v = {0u, 0u, 0u, 0u};
            if (r < rows)
                v = *reinterpret_cast<const u32x4_t*>(
                    qrot + ((int64_t)(t.tok0 + r / G) * H + kvh * G + r % G) * HD + c * 8);
            *reinterpret_cast<u32x4_t*>(&sQ[r * KP + c * 8]) = v ^ qsign;
        }
    }
    float m = -INFINITY;
    float16_t oT[DT];
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int e = 0; e < 16; ++e) oT[d][e] = 0.f;
    // Running softmax sum over this lane's keys (its 32 of each 64-key block); the
    // two lanes of a query add theirs at the end.
    float lsum = 0.f;

    constexpr int KPT = kKeyTile * (HD / 8) / NT, VPT = kKeyTile * (VHD / 8) / NT;
    static_assert(KPT >= 1 && VPT >= 1, "block staging");
    // Native vectors, not uint4: a struct-typed copy keeps these arrays in memory
    // (the compiler moved them to LDS or scratch, and waited on every prefetch to
    // store it there); as vectors they stay in registers.
    u32x4_t kreg[KPT], vreg[VPT];
    int kok = 0, vok = 0;
    // Paged rows: the block-table entries of keys [k0, min(k1, past)) are staged in
    // LDS once, as the cache row index of row 0 of (block, kv head), phys * blk * KV
    // + kvh, or ~0u for an entry out of range; a row then costs an LDS read, a
    // shift (a division for block sizes that are not powers of two) and 32-bit
    // integer work. A range of more than kBtLds blocks, or a cache of 2^32 rows
    // or more, reads the table from global memory instead (the second form of the
    // walk below).
    constexpr int kBtLds = 512;
    __shared__ uint32_t s_bt[PAGED ? kBtLds : 1];
    int lb0 = 0;
    bool bt_lds = true;
    if constexpr (PAGED) {
        const int cend = min(k1, t.past);
        if (cend > k0) {
            lb0 = k0 / pk.blk;
            const int n = (cend - 1) / pk.blk - lb0 + 1;
            bt_lds = n <= kBtLds && pk.nblk * pk.blk * pk.KV < (int64_t)0xffffffff;
            if (bt_lds)
                for (int i = tid; i < n; i += NT) {
                    const int lb = lb0 + i;
                    const int phys = lb < pk.maxb ? pk.bt[(int64_t)t.seq * pk.maxb + lb] : -1;
                    s_bt[i] = phys >= 0 && phys < pk.nblk
                                  ? ((uint32_t)phys * (uint32_t)pk.blk) * (uint32_t)pk.KV + kvh
                                  : ~0u;
                }
        }
        __syncthreads();
    }
    // Byte address of new row 0 of the sequence's (virtual) new-row range, such
    // that key j >= past is at nrow0 + j * nstride (modular arithmetic).
    // Cache and new rows, keys and values alike, are HD dims apart: with a value
    // cache VHD equals HD (the entry point checks it), and without one the values
    // are the leading VHD dims of the key rows.
    constexpr uint32_t kRowBytes = HD * 2;
    // (Pointer arithmetic, not integers, so the loads stay global loads: a flat
    // load would also count against every LDS wait.)
    const uint32_t nstride = (uint32_t)pk.KV * HD * 2;
    const int64_t nrow0 = ((int64_t)(t.tok_seq0 - t.past) * pk.KV + kvh) * HD * 2;
    const char* nrow_k = static_cast<const char*>(pk.knew) + nrow0;
    const char* nrow_v = static_cast<const char*>(pk.vnew ? pk.vnew : pk.knew) + nrow0;
    // Source row of key j (k0 <= j < k1): always a valid address; `ok` is false
    // for a row whose block-table entry is out of range (block 0 stands in). Both
    // candidates (the sequence's new row, the cache row) are formed and one is
    // selected, with no branch. With the table in LDS (`lds` true) forming an
    // address issues no global load: a global load between two K/V loads would
    // make the wait for its table entry wait for the K/V loads issued before it
    // (loads retire in order), and the block's loads would run one at a time.
    auto row_src = [&](int j, bool value, bool& ok, auto lds) -> const half_t* {
        if constexpr (!PAGED) {
            ok = true;
            const half_t* base = static_cast<const half_t*>(value ? dk.v : dk.k);
            return base + (((int64_t)t.seq * dk.KV + kvh) * dk.cap + j) * (value ? VHD : HD);
        } else {
            const bool fresh = j >= t.past;
            const int jc = fresh ? k0 : j;  // a cache row stands in for a new one
            int lb, within;
            if (pk.blk_shift >= 0) {
                lb = jc >> pk.blk_shift;
                within = jc & ((1 << pk.blk_shift) - 1);
            } else {
                lb = jc / pk.blk;
                within = jc - lb * pk.blk;
            }
            const char* ac;
            bool cok;
            if constexpr (decltype(lds)::value) {
                const uint32_t e = s_bt[min((unsigned)(lb - lb0), (unsigned)(kBtLds - 1))];
                cok = e != ~0u;
                const uint32_t r = (cok ? e : 0u) + __umul24((uint32_t)within, (uint32_t)pk.KV);
                const char* cb = static_cast<const char*>((value && pk.vcache) ? pk.vcache : pk.kcache);
                ac = cb + (uint64_t)r * kRowBytes;
            } else {
                // maxb >= 1 (the entry point checks it), so the clamped index is in range.
                const int e = pk.bt[(int64_t)t.seq * pk.maxb + min(lb, pk.maxb - 1)];
                const int phys = lb < pk.maxb ? e : -1;
                cok = phys >= 0 && phys < pk.nblk;
                const int64_t slot = (int64_t)(cok ? phys : 0) * pk.blk + within;
                const char* cb = static_cast<const char*>((value && pk.vcache) ? pk.vcache : pk.kcache);
                ac = cb + (uint64_t)(slot * pk.KV + kvh) * kRowBytes;
            }
            const char* an = (value ? nrow_v : nrow_k) + (uint64_t)(uint32_t)j * (uint64_t)nstride;
            ok = fresh || cok;
            return reinterpret_cast<const half_t*>(fresh ? an : ac);
        }
    };
    // A 64-key block into registers, keys and values separately: the row addresses
    // first, then the loads back to back. Loads are never conditional (a branch
    // around a load makes the compiler drain every prefetch at the join): rows past
    // the block end load its last row again, and the validity bits mask keys (sOk)
    // and zero values at commit. A thread stages one key row (NT is a multiple of
    // the block) and VPT consecutive value rows of one 8-dim chunk, so the
    // transposed store writes VPT keys of a head dim at once.
    static_assert(NT % kKeyTile == 0, "one key row per thread");
    auto fetch_k = [&](int kb, auto lds) {
        const int nk = min(kKeyTile, k1 - kb);
        const int rk = tid % kKeyTile;
        bool okk;
        const half_t* pkr = row_src(kb + min(rk, nk - 1), false, okk, lds);
#pragma unroll
        for (int i = 0; i < KPT; ++i)
            kreg[i] = *reinterpret_cast<const u32x4_t*>(pkr + ((tid + NT * i) / kKeyTile) * 8);
        kok = okk && rk < nk;
    };
    auto fetch_v = [&](int kb, auto lds) {
        const int nk = min(kKeyTile, k1 - kb);
        const int rv = VPT * (tid % (kKeyTile / VPT)), cv = (tid / (kKeyTile / VPT)) * 8;
        bool okv[VPT];
        const half_t* pvr[VPT];
#pragma unroll
        for (int i = 0; i < VPT; ++i) pvr[i] = row_src(kb + min(rv + i, nk - 1), true, okv[i], lds);
#pragma unroll
        for (int i = 0; i < VPT; ++i) vreg[i] = *reinterpret_cast<const u32x4_t*>(pvr[i] + cv);
        vok = 0;
#pragma unroll
        for (int i = 0; i < VPT; ++i) vok |= (int)(okv[i] && rv + i < nk) << i;
    };
    auto commit_k = [&]() {
#pragma unroll
        for (int i = 0; i < KPT; ++i) {
            const int idx = tid + NT * i, r = idx % kKeyTile, c = (idx / kKeyTile) * 8;
            *reinterpret_cast<u32x4_t*>(&sK[r * KP + c]) = kreg[i];
        }
        // Threads 0..63 hold the first vector (c = 0) of keys 0..63: one ballot.
        const unsigned long long ok = __ballot(kok & 1);
        if (tid == 0) sOk = ok;
    };
    auto commit_v = [&]() {
        const int r0 = VPT * (tid % (kKeyTile / VPT)), c = (tid / (kKeyTile / VPT)) * 8;
#pragma unroll
        for (int i = 0; i < VPT; ++i)
            if (!((vok >> i) & 1)) vreg[i] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            uint16_t col[VPT];
#pragma unroll
            for (int i = 0; i < VPT; ++i) col[i] = __builtin_bit_cast(u16x8_t, vreg[i])[e];
            if constexpr (VPT == 4)
                *reinterpret_cast<uint2*>(&sVt[(c + e) * VP + r0]) =
                    *reinterpret_cast<const uint2*>(col);
            else if constexpr (VPT == 2)
                *reinterpret_cast<uint32_t*>(&sVt[(c + e) * VP + r0]) =
                    *reinterpret_cast<const uint32_t*>(col);
            else
#pragma unroll
                for (int i = 0; i < VPT; ++i) sVt[(c + e) * VP + r0 + i] = col[i];
        }
    };
    // S^T of the staged keys against this wave's queries (two 32-key tiles).
    auto scores = [&](float16_t (&st)[2]) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int e = 0; e < 16; ++e) st[kt][e] = 0.f;
#pragma unroll
        for (int s2 = 0; s2 < HD / 16; ++s2)
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                const u16x8_t a =
                    *reinterpret_cast<const u16x8_t*>(&sK[(kt * 32 + lrow) * KP + s2 * 16 + lk]);
                const u16x8_t b = *reinterpret_cast<const u16x8_t*>(&sQ[q * KP + s2 * 16 + lk]);
                st[kt] = tile_mfma<T>(a, b, st[kt]);
            }
    };
    // The key walk, software-pipelined across blocks: while the matrix cores score
    // block b + 1, the vector units run the softmax of block b, whose scores came
    // from the previous step. Keys are therefore staged one block ahead of values:
    // a step commits V(b) and K(b + 1), both into slots whose last readers finished
    // before the previous barrier. Per-block work is unchanged; only its order is.
    auto walk = [&](auto lds) {
        if (k0 >= k1) return;
        fetch_k(k0, lds);
        fetch_v(k0, lds);
        commit_k();
        __syncthreads();
        unsigned long long okm = sOk;
        if (k0 + kKeyTile < k1) fetch_k(k0 + kKeyTile, lds);
        float16_t stA[2], stB[2];
        scores(stA);
        __syncthreads();  // sK is restaged by the first step
        auto step = [&](int kb, float16_t (&cur)[2], float16_t (&nxt)[2]) {
            const bool more = kb + kKeyTile < k1;
            commit_v();
            if (more) commit_k();
            __syncthreads();
            const unsigned long long okm_next = sOk;
            if (more) {
                fetch_v(kb + kKeyTile, lds);
                if (kb + 2 * kKeyTile < k1) fetch_k(kb + 2 * kKeyTile, lds);
            }
            // Keys of block kb that are out of range, causally hidden or behind an
            // invalid block-table entry (only blocks that are not fully visible).
            const bool full = kb + kKeyTile <= k1 && okm == ~0ull && kb + kKeyTile - 1 <= qpos_wave;
            if (!full) {
#pragma unroll
                for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int kk = kt * 32 + 8 * (e / 4) + 4 * hh + (e & 3);
                        const int j = kb + kk;
                        const bool ok = j < k1 && j <= qpos && ((okm >> kk) & 1ull);
                        cur[kt][e] = ok ? cur[kt][e] : -INFINITY;
                    }
            }
            if (more) scores(nxt);
            // Block max of the raw scores. Scaling by sc2 > 0 keeps the maximum (and
            // rounds it alike), so the scale joins the exponent's argument in one fma.
            float bmax = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 16; ++e) bmax = fmaxf(bmax, cur[kt][e]);
            {
                const LanePair pr = swap32(bmax);
                bmax = fmaxf(pr.a, pr.b);
            }
            // The reference point m moves only when the block max passes it by more
            // than kLazy (log2 units), so P = exp2(s - m) stays below 2^kLazy (exact
            // in fp16's range) and O is rarely rescaled; the final O / l, and the
            // merge of (m, l, O) partials, do not depend on where m sits.
            constexpr float kLazy = 8.f;
            const float bm = bmax * sc2;
            const float m_new = bm > m + kLazy ? bm : m;
            // v_exp_f32 directly: results below 2^-126 flush to zero, which the
            // softmax weights can afford.
            const float alpha = (m == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
            // P^T operands: k-step kk uses e in [8 (kk % 2), 8 (kk % 2) + 8) of tile kk / 2.
            u16x8_t pb[4];
            const float mref = m_new == -INFINITY ? 0.f : m_new;  // exp2(-inf - 0) = 0
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    pb[kt * 2 + e / 8][e % 8] =
                        tile_round<T>(__builtin_amdgcn_exp2f(fmaf(cur[kt][e], sc2, -mref)));
            m = m_new;
            // Rescale O (and the running sums) only when some query's running max moved.
            if (__any(alpha != 1.f)) {
#pragma unroll
                for (int d = 0; d < DT; ++d)
#pragma unroll
                    for (int e = 0; e < 16; ++e) oT[d][e] *= alpha;
            }
            // Row sums of the same rounded probabilities that weight V, accumulated in
            // fp32 (v_dot2 against ones, four independent chains).
            {
                float ls[4];
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    ls[kk] = 0.f;
                    const u32x4_t pw = __builtin_bit_cast(u32x4_t, pb[kk]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) ls[kk] = tile_pair_sum<T>(pw[i], ls[kk]);
                }
                lsum = fmaf(lsum, alpha, (ls[0] + ls[1]) + (ls[2] + ls[3]));
            }
            // O^T += V^T P^T over the 4 k-steps of 16 keys.
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int kbase = (kk / 2) * 32 + (kk % 2) * 16 + 4 * hh;
#pragma unroll
                for (int d = 0; d < DT; ++d) {
                    const uint16_t* vr = &sVt[(d * 32 + lrow) * VP + kbase];
                    const u32x2_t lo = *reinterpret_cast<const u32x2_t*>(vr);
                    const u32x2_t hi = *reinterpret_cast<const u32x2_t*>(vr + 8);
                    const u16x8_t a = __builtin_bit_cast(u16x8_t, u32x4_t{lo[0], lo[1], hi[0], hi[1]});
                    oT[d] = tile_mfma<T>(a, pb[kk], oT[d]);
                }
            }
            okm = okm_next;
            __syncthreads();  // the next step restages sK, sVt and sOk
        };
        for (int kb = k0; kb < k1; kb += 2 * kKeyTile) {
            step(kb, stA, stB);
            if (kb + kKeyTile < k1) step(kb + kKeyTile, stB, stA);
        }
    };
    if (bt_lds)
        walk(std::true_type{});
    else
        walk(std::false_type{});
    {
        const LanePair pr = swap32(lsum);
        lsum = pr.a + pr.b;
    }
    if (!qlive) return;
    float l = lsum;
    m = m == -INFINITY ? m : m / kLog2e;  // back to the natural-log domain of the merge
    const int tok = t.tok0 + q / G, h = kvh * G + q % G;
    if (part) {
        float* dst = part + (((int64_t)tok * H + h) * nsplit + split) * (VHD + 2);
#pragma unroll
        for (int d = 0; d < DT; ++d)
#pragma unroll
            for (int e = 0; e < 16; ++e) dst[d * 32 + 8 * (e / 4) + 4 * hh + (e & 3)] = oT[d][e];
        if (hh == 0) {
            dst[VHD] = m;
            dst[VHD + 1] = l;
        }
        return;
    }
    float a = 1.f;
    if (sink) {
        const float sv2 = sink[h];
        const float mm = fmaxf(m, sv2);
        a = (m == -INFINITY) ? 0.f : __expf(m - mm);
        l = l * a + __expf(sv2 - mm);
    }
    const float inv = l > 0.f ? a / l : 0.f;
    T* dst = out + (int64_t)tok * out_tok_stride + (int64_t)h * VHD;
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
            uint16_t v4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v4[i] = tile_round<T>(oT[d][4 * e4 + i] * inv);
            *reinterpret_cast<uint2*>(dst + d * 32 + 8 * e4 + 4 * hh) =
                *reinterpret_cast<const uint2*>(v4);
        }
}

// Tile body for a dtype: the matrix-core tile for fp16 and bf16 (NW waves of 32
// query rows), the VALU tile (kTileRows rows, 256 threads) otherwise.
template <typename T, int VHD>
constexpr bool mfma_tile() {
    return (std::is_same<T, half_t>::value || std::is_same<T, uint16_t>::value) && VHD % 32 == 0;
}
// Query rows per workgroup of the tile body used for dtype T.
template <typename T>
static int tile_rows_for(int vhd, int nw = 4) {
    return (std::is_same<T, half_t>::value || std::is_same<T, uint16_t>::value) && vhd % 32 == 0
               ? 32 * nw
               : kTileRows;
}
// Threads of a tile workgroup.
template <typename T, int VHD, int NW>
constexpr int tile_threads() {
    return mfma_tile<T, VHD>() ? 64 * NW : 256;
}

template <typename T, int HD, int VHD, bool PAGED, int NW = 4>
__device__ __forceinline__ void attn_tile(const TileDesc& t, int kvh, int G, int H,
                                          const T* __restrict__ qrot, const DenseKV& dk,
                                          const PagedKV& pk, float scale,
                                          const float* __restrict__ sink, int k0, int k1,
                                          T* __restrict__ out, int64_t out_tok_stride,
                                          float* __restrict__ part, int nsplit, int split) {
    if constexpr (mfma_tile<T, VHD>())
        attn_mfma_body<T, HD, VHD, PAGED, NW>(t, kvh, G, H, qrot, dk, pk, scale, sink, k0, k1, out,
                                            out_tok_stride, part, nsplit, split);
    else
        attn_tile_body<T, HD, VHD, PAGED>(t, kvh, G, H, qrot, dk, pk, scale, sink, k0, k1, out,
                                          out_tok_stride, part, nsplit, split);
}

// GQA prefill / S > 1: grid (B * tiles_per_seq, KV). Keys from `present`. The
// matrix-core tile takes 8 waves (256 query rows, one workgroup per CU), as the
// paged tile does: the per-thread K/V prefetch halves, which keeps the body
// within 256 VGPRs.
constexpr int kGqaTileWaves = 8;
template <typename T, int HD>
__global__ __launch_bounds__((tile_threads<T, HD, kGqaTileWaves>()),
                             (mfma_tile<T, HD>() ? 1 : 2)) void gqa_tile_kernel(const T* __restrict__ qrot, DenseKV dk,
                                                       int S, int QT, int tiles_per_seq, int G,
                                                       int H, int vp, float scale,
                                                       T* __restrict__ out, int chunk, int nsplit,
                                                       float* __restrict__ part,
                                                       int* __restrict__ nsplit_row) {
    const int b = blockIdx.x / tiles_per_seq;
    const int tile = blockIdx.x % tiles_per_seq;
    const int kvh = blockIdx.y, split = blockIdx.z;
    TileDesc t;
    t.seq = b;
    const int s0 = tile * QT;
    t.ntok = min(QT, S - s0);
    t.tok0 = b * S + s0;
    t.qpos0 = vp + s0;
    t.past = vp;
    t.nkeys = vp + S;
    t.tok_seq0 = b * S;
    PagedKV none{};
    const int k1 = min(t.nkeys, t.qpos0 + t.ntok);  // causal bound of the tile
    // Key splits of `chunk` keys (the last takes the rest); rows of a tile that
    // needs one split are written directly and marked 0 for the merge.
    const int ns = min(nsplit, max(1, (k1 + chunk - 1) / chunk));
    if (split == 0 && nsplit > 1) {
        for (int r = threadIdx.x; r < t.ntok * G; r += blockDim.x)
            nsplit_row[(int64_t)(t.tok0 + r / G) * H + kvh * G + r % G] = ns > 1 ? ns : 0;
    }
    if (split >= ns) return;
    if (ns == 1) {
        attn_tile<T, HD, HD, false, kGqaTileWaves>(t, kvh, G, H, qrot, dk, none, scale, nullptr,
                                                   0, k1, out, (int64_t)H * HD, nullptr, 1, 0);
        return;
    }
    const int k0 = split * chunk;
    const int ks1 = split == ns - 1 ? k1 : min(k1, k0 + chunk);
    attn_tile<T, HD, HD, false, kGqaTileWaves>(t, kvh, G, H, qrot, dk, none, scale, nullptr, k0,
                                               ks1, out, (int64_t)H * HD, part, nsplit, split);
}

// ------------------------------------------------------- PagedAttention --

// Tile map built on the device by one 64-lane wave (no host read of the control
// tensors): ceil(n_b / QT) tiles of QT tokens for each sequence b, in sequence
// order, tiles[i] = {seq, first token, ntok, first token of the sequence}, and
// the count. Token ranges are clamped to [0, T), so a malformed cum_seqlens
// yields fewer tiles, never a tile outside the batch, and the attention kernels
// take the sequence start from the tile (clamped) rather than from cum_seqlens:
// a new key row is then always a token of [0, T). At most max_tiles are written.
__device__ void build_tile_map(const int32_t* __restrict__ cum, int batch, int T, int QT,
                               int max_tiles, int4* __restrict__ tiles, int* __restrict__ count) {
    const int lane = threadIdx.x;
    int base = 0;
    for (int b0 = 0; b0 < batch; b0 += 64) {
        const int b = b0 + lane;
        int s0 = 0, s1 = 0;
        if (b < batch) {
            s0 = min(max(cum[b], 0), T);
            s1 = min(max(cum[b + 1], s0), T);
        }
        const int nt = (s1 - s0 + QT - 1) / QT;
        int incl = nt;  // inclusive prefix sum of the tile counts over the wave
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o, 64);
            if (lane >= o) incl += v;
        }
        const int first = base + incl - nt;
        for (int i = 0; i < nt && first + i < max_tiles; ++i) {
            const int t = s0 + i * QT;
            tiles[first + i] = make_int4(b, t, min(QT, s1 - t), s0);
        }
        base += __shfl(incl, 63, 64);
    }
    if (lane == 0) *count = min(base, max_tiles);
}

// One workgroup (64 threads) per (token, head slot); slots 0..H-1 are query
// heads, H..H+KV-1 key heads. Q/K: optional RMS norm, RoPE; rotated Q ->
// qrot, rotated K -> knew, K/V -> cache slot.
template <typename T>
__global__ __launch_bounds__(64 * kPrepHeads) void paged_prep_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    T* __restrict__ kcache, T* __restrict__ vcache, int64_t nblk, int blk,
    const int32_t* __restrict__ cum, const int32_t* __restrict__ past,
    const int32_t* __restrict__ bt, int batch, int maxb, const T* __restrict__ cos_c,
    const T* __restrict__ sin_c, int half, int interleaved, int rot_off,
    const int32_t* __restrict__ slot_mapping, const T* __restrict__ qw,
    const T* __restrict__ kw, float eps, int H, int KV, int hd, int vhd,
    T* __restrict__ qrot, T* __restrict__ knew, int64_t max_pos, int QT, int max_tiles,
    int4* __restrict__ tiles, int* __restrict__ tile_count, int* __restrict__ nsplit_row) {
    extern __shared__ float sv_all[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // One wave per (token, head), kPrepHeads heads per workgroup.
    const int tok = blockIdx.x, head = blockIdx.y * kPrepHeads + wave;
    if (head >= H + KV) return;
    float* sv = sv_all + wave * hd;
    // Two jobs for the attention kernels that follow, folded in to save launches:
    // block (0, 0) builds the tile map, and each query row's split count starts
    // at 0 (a row no tile owns, under a malformed cum_seqlens, keeps it).
    if (tok == 0 && head == 0)
        build_tile_map(cum, batch, (int)gridDim.x, QT, max_tiles, tiles, tile_count);
    if (head < H && lane == 0) nsplit_row[(int64_t)tok * H + head] = 0;
    const bool is_q = head < H;
    const T* src = is_q ? q + ((int64_t)tok * H + head) * hd
                        : k + ((int64_t)tok * KV + (head - H)) * hd;
    // Sequence of this token: the last b with cum[b] <= tok. Up to 64 sequences,
    // lane l holds cum[l] and past[l] (one batch of loads, together with the
    // head row) and a ballot counts the cum[l] <= tok for l >= 1; beyond that, a
    // binary search.
    int b, cb, pb;
    if (batch <= 64) {
        const int l = min(lane, batch - 1);
        const int cl = cum[l], pl = past[l];
        row_to_lds<T>(sv, src, hd, lane);
        b = (int)__popcll(__ballot(lane >= 1 && lane < batch && cl <= tok));
        cb = __shfl(cl, b, 64);
        pb = __shfl(pl, b, 64);
    } else {
        int lo = 0, hi = batch;  // invariant: cum[lo] <= tok < cum[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) / 2;
            if (cum[mid] <= tok) lo = mid;
            else hi = mid;
        }
        b = lo;
        cb = cum[b];
        pb = past[b];
        row_to_lds<T>(sv, src, hd, lane);
    }
    // The sequence start clamped to [0, T), as the tile map and the attention
    // kernels take it, so positions agree across the kernels of one call.
    // past is clamped below at 0 as there, and the position is formed in 64 bits
    // (a past near 2^31 then gives a position past the block table, not a wrap).
    cb = min(max(cb, 0), (int)gridDim.x);
    const int pos = (int)min((int64_t)max(pb, 0) + (tok - cb), (int64_t)INT32_MAX);
    const T* nw = is_q ? qw : kw;
    if (nw) rms_head_lds<T>(sv, hd, nw, eps);
    if (cos_c) {
        // A position outside the cache violates the op contract; clamp the row so
        // the read stays inside the cos/sin tensors.
        const int64_t prow = pos < 0 ? 0 : (pos >= max_pos ? max_pos - 1 : pos);
        rope_head_lds<T>(sv, cos_c + prow * half, sin_c + prow * half, half, interleaved, rot_off);
        for (int d = lane; d < hd; d += 64) sv[d] = round_to<T>(sv[d]);
    }
    if (is_q) {
        lds_to_row<T>(qrot + ((int64_t)tok * H + head) * hd, sv, hd, lane);
        return;
    }
    const int kvh = head - H;
    lds_to_row<T>(knew + ((int64_t)tok * KV + kvh) * hd, sv, hd, lane);
    int64_t slot;
    if (slot_mapping) {
        slot = slot_mapping[tok];
    } else {
        const int lb = pos / blk;
        const int phys = (pos >= 0 && lb < maxb) ? bt[(int64_t)b * maxb + lb] : -1;
        slot = phys < 0 ? -1 : (int64_t)phys * blk + pos % blk;
    }
    if (slot < 0 || slot >= nblk * blk) return;
    lds_to_row<T>(kcache + (slot * KV + kvh) * hd, sv, hd, lane);
    if (vcache) {
        copy_row<T>(vcache + (slot * KV + kvh) * vhd, v + ((int64_t)tok * KV + kvh) * vhd, vhd,
                    lane);
    }
}

// grid (max_tiles, KV, nsplit). A tile's causal key range [0, kend) is split
// into `chunk`-key ranges; with one range the tile writes its rows directly,
// otherwise each split writes partial rows (token-major, row tok * H + h) and
// split 0 records the split count of its rows for paged_merge (0 = direct).
// Two workgroups per CU (launch bound): a few VGPRs spill, but the second wave per
// SIMD hides the K/V fetch of the first (mixed 32-sequence batch 917 -> 756 us).
// Paged prefill tiles take 8 waves (256 query rows) on the matrix-core path: each
// K/V block fetched serves twice the queries of a 4-wave tile.
constexpr int kPagedTileWaves = 8;
template <typename T, int HD, int VHD>
__global__ __launch_bounds__((tile_threads<T, VHD, kPagedTileWaves>()),
                             (mfma_tile<T, VHD>() ? 1 : 2)) void paged_tile_kernel(
    const int4* __restrict__ tiles, const int* __restrict__ tile_count,
    const int32_t* __restrict__ cum, const int32_t* __restrict__ past_lens, PagedKV pk,
    const T* __restrict__ qrot, int G, int H, float scale, const float* __restrict__ sink,
    int chunk, int nsplit, T* __restrict__ out, float* __restrict__ part,
    int* __restrict__ nsplit_row, int skip_single, int mt) {
    // The tiles of one (kv head, split) group read the same K/V rows. Groups
    // gi = kvh + KV * split are dealt round-robin to the XCDs, and an XCD runs
    // all mt tile slots of a group back to back, so those reads meet in its L2.
    // Dealing by gi % kXcds mixes splits on every XCD (late splits are often
    // empty). Grid: kXcds * mt * ceil(KV * nsplit / kXcds) workgroups.
    const int xcd = (int)blockIdx.x % kXcds, slot = (int)blockIdx.x / kXcds;
    const int gi = xcd + kXcds * (slot / mt), ti = slot % mt;
    const int kvh = gi % pk.KV, split = gi / pk.KV;
    if (split >= nsplit || ti >= *tile_count) return;
    const int4 td = tiles[ti];
    if (skip_single && td.z == 1) return;  // paged_decode_kernel's
    TileDesc t;
    t.seq = td.x;
    t.tok0 = td.y;
    t.ntok = td.z;
    // Sequence start from the tile map (clamped to the batch); past clamped to
    // [0, max_ctx], so every new key row is a token of the tile's sequence range
    // and the walk is bounded whatever past_seqlens holds.
    t.tok_seq0 = td.w;
    t.past = min(max(past_lens[t.seq], 0), pk.max_ctx);
    t.qpos0 = t.past + (t.tok0 - t.tok_seq0);
    t.nkeys = t.qpos0 + t.ntok;
    const int kend = min(t.nkeys, pk.max_ctx);  // causal bound of the tile
    DenseKV none{};
    const int ns = min(nsplit, max(1, (kend + chunk - 1) / chunk));
    if (split == 0) {
        for (int r = threadIdx.x; r < t.ntok * G; r += blockDim.x)
            nsplit_row[(int64_t)(t.tok0 + r / G) * H + kvh * G + r % G] = ns > 1 ? ns : 0;
    }
    if (split >= ns) return;
    if (ns == 1) {
        attn_tile<T, HD, VHD, true, kPagedTileWaves>(t, kvh, G, H, qrot, none, pk, scale, sink, 0, kend, out,
                                    (int64_t)H * VHD, nullptr, 1, 0);
        return;
    }
    const int k0 = split * chunk;
    const int k1 = split == ns - 1 ? kend : min(kend, k0 + chunk);
    attn_tile<T, HD, VHD, true, kPagedTileWaves>(t, kvh, G, H, qrot, none, pk, scale, sink, k0, k1, out,
                                (int64_t)H * VHD, part, nsplit, split);
}

// Single-token tiles (every decoding sequence, and the last token of a prefill
// whose length leaves one over) on the vector units, the way the dense decode
// kernel does them: the G query heads of one kv head against keys [k0, k1) of the
// sequence, one 16-byte slice of a key/value row per lane, rows spread over lane
// groups, a blocked online softmax and loads one block ahead. Cache rows are
// found through the block table, whose slice for the keys in hand is staged in
// LDS first; rows from `past` on are the sequence's own new (rotated) keys and
// values. A row whose block-table entry is out of range is masked, as in the tile
// kernel. grid (max_tiles, KV, nsplit), same splits and outputs as
// paged_tile_kernel, which leaves these tiles to this kernel.
template <typename T, int HD, int G>
__global__ __launch_bounds__(256) void paged_decode_kernel(
    const int4* __restrict__ tiles, const int* __restrict__ tile_count,
    const int32_t* __restrict__ cum, const int32_t* __restrict__ past_lens, PagedKV pk,
    int blk_shift, const T* __restrict__ qrot, int H, float scale,
    const float* __restrict__ sink, int chunk, int nsplit, T* __restrict__ out,
    float* __restrict__ part, int* __restrict__ nsplit_row) {
    constexpr int LPR = HD / 8;        // lanes per row (16 bytes each)
    constexpr int RPW = 64 / LPR;      // rows per wave per step
    constexpr int RPS = 4 * RPW;       // rows per workgroup step
    constexpr int U = G <= 4 ? 4 : 2;  // steps per online-softmax block
    constexpr int BLK = RPS * U;       // rows per block
    constexpr int kBt = 256;           // block-table entries staged at a time
    __shared__ int s_bt[kBt];
    __shared__ float s_o[4][G][HD];
    __shared__ float s_m[4][G], s_l[4][G];

    const int ti = blockIdx.x, kvh = blockIdx.y, split = blockIdx.z;
    if (ti >= *tile_count) return;
    const int4 td = tiles[ti];
    if (td.z != 1) return;
    const int seq = td.x, tok = td.y;
    const int tok_seq0 = td.w;  // clamped sequence start (tile map)
    const int past = min(max(past_lens[seq], 0), pk.max_ctx);
    // causal: keys up to the token itself, none at positions >= max_ctx
    const int kend = min(past + (tok - tok_seq0) + 1, pk.max_ctx);
    const int ns = min(nsplit, max(1, (kend + chunk - 1) / chunk));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int sub = lane / LPR;
    const int dl = (lane % LPR) * 8;
    const int KV = pk.KV;
    if (split == 0 && tid < G) nsplit_row[(int64_t)tok * H + kvh * G + tid] = ns > 1 ? ns : 0;
    if (split >= ns) return;
    const int k0 = split * chunk;
    const int k1 = split == ns - 1 ? kend : min(kend, k0 + chunk);

    const T* kc = static_cast<const T*>(pk.kcache) + (int64_t)kvh * HD + dl;
    const T* vc = static_cast<const T*>(pk.vcache) + (int64_t)kvh * HD + dl;
    // New rows: row past + i is token tok_seq0 + i.
    const int64_t new0 = (int64_t)tok_seq0 - past;
    const T* kn = static_cast<const T*>(pk.knew) + (int64_t)kvh * HD + dl;
    const T* vn = static_cast<const T*>(pk.vnew) + (int64_t)kvh * HD + dl;
    const int64_t rs = (int64_t)KV * HD;  // row stride of caches and new rows
    const int bmask = (1 << blk_shift) - 1;

    // Scores are raw dot products with the rotated query; the softmax scale (and
    // log2 e, for the hardware exp2) is applied inside the exponent. fp16 rows
    // take two dims per v_dot2_f32_f16 (exact products, fp32 accumulation).
    constexpr bool kDot2 = std::is_same<T, half_t>::value;
    uint4 qraw[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
        qraw[g] = *reinterpret_cast<const uint4*>(qrot + ((int64_t)tok * H + kvh * G + g) * HD + dl);
    auto qk = [&](int g, const uint4& kv) -> float {
        float d = 0.f;
        if constexpr (kDot2) {
            const uint32_t qw[4] = {qraw[g].x, qraw[g].y, qraw[g].z, qraw[g].w};
            const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
            for (int p = 0; p < 4; ++p)
                d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, qw[p]),
                                           __builtin_bit_cast(half2_t, kw[p]), d, false);
        } else {
            const T* qt = reinterpret_cast<const T*>(&qraw[g]);
            const T* kt = reinterpret_cast<const T*>(&kv);
#pragma unroll
            for (int i = 0; i < 8; ++i) d = fmaf(to_f32(qt[i]), to_f32(kt[i]), d);
        }
        return d;
    };
    constexpr float kLog2e = 1.4426950408889634f;
    const float c2 = scale * kLog2e;
    float m[G], l[G], o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) o[g][i] = 0.f;
    }

    // Windows [w0, w1) of keys whose block-table slice fits s_bt: (kBt - 1) blocks
    // of keys touch at most kBt blocks whatever the alignment of w0.
    const int W = (kBt - 1) << blk_shift;
    for (int w0 = k0; w0 < k1; w0 += W) {
        const int w1 = min(k1, w0 + W);
        const int lb0 = w0 >> blk_shift;
        const int cend = min(w1, past);  // cache rows are [w0, cend)
        const int nlb = cend > w0 ? ((cend - 1) >> blk_shift) - lb0 + 1 : 0;
        if (w0 != k0) __syncthreads();  // the previous window is done with s_bt
        for (int i = tid; i < nlb; i += 256) {
            const int lb = lb0 + i;
            s_bt[i] = lb < pk.maxb ? pk.bt[(int64_t)seq * pk.maxb + lb] : -1;
        }
        __syncthreads();

        // Rows beyond w1 load row w1 - 1 again (masked); a row with a bad
        // block-table entry loads row 0 of block 0 (masked, value zeroed).
        uint4 kr[U], vr[U];
        unsigned okr = 0;
        auto load_block = [&](uint4 (&kk)[U], uint4 (&vv)[U], unsigned& ok, int base) {
            ok = 0;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = min(base + u * RPS + wave * RPW + sub, w1 - 1);
                const bool cached = j < past;
                const int phys = s_bt[cached ? (j >> blk_shift) - lb0 : 0];
                const bool good = !cached || (phys >= 0 && phys < pk.nblk);
                const int64_t slot = good ? (int64_t)phys * (bmask + 1) + (j & bmask) : 0;
                const T* kp = cached ? kc + slot * rs : kn + (new0 + j) * rs;
                const T* vp = cached ? vc + slot * rs : vn + (new0 + j) * rs;
                // Streamed once per step: non-temporal.
                const u32x4_t kq = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(kp));
                const u32x4_t vq = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(vp));
                kk[u] = make_uint4(kq.x, kq.y, kq.z, kq.w);
                vv[u] = make_uint4(vq.x, vq.y, vq.z, vq.w);
                ok |= (unsigned)good << u;
            }
        };
        auto process = [&](const uint4 (&kk)[U], const uint4 (&vv)[U], unsigned ok, int base) {
            float sc[U][G];
            float bmax[G];
#pragma unroll
            for (int g = 0; g < G; ++g) bmax[g] = -INFINITY;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int j = base + u * RPS + wave * RPW + sub;
                const bool live = j < w1 && ((ok >> u) & 1u);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float d = group_sum<LPR>(qk(g, kk[u]));
                    sc[u][g] = live ? d : -INFINITY;
                    bmax[g] = fmaxf(bmax[g], sc[u][g]);
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float mn = fmaxf(m[g], bmax[g]);
                // m = -inf (nothing seen yet) gives alpha 0; mn = -inf keeps everything 0.
                const float alpha =
                    m[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m[g] - mn) * c2);
                l[g] *= alpha;
#pragma unroll
                for (int i = 0; i < 8; ++i) o[g][i] *= alpha;
                m[g] = mn;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const bool good = (ok >> u) & 1u;
                const T* vv8 = reinterpret_cast<const T*>(&vv[u]);
                float vf[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) vf[i] = good ? to_f32(vv8[i]) : 0.f;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = sc[u][g] == -INFINITY
                                        ? 0.f
                                        : __builtin_amdgcn_exp2f(fmaf(sc[u][g], c2, -m[g] * c2));
                    l[g] += p;
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[g][i] = fmaf(p, vf[i], o[g][i]);
                }
            }
        };
        // The next block is always requested (rows past w1 repeat row w1 - 1): a
        // load behind a branch would make the compiler wait for every load in
        // flight where the paths join. The loop takes blocks in pairs with no exit
        // inside its body (an odd count ends with one fully masked block): with a
        // mid-body exit the compiler copied the register sets between iterations,
        // and a copy of a register still being loaded waited for every load in
        // flight, the prefetched block included.
        uint4 kn2[U], vn2[U];
        unsigned okn = 0;
        load_block(kr, vr, okr, w0);
        for (int base = w0; base < w1; base += 2 * BLK) {
            load_block(kn2, vn2, okn, base + BLK);
            process(kr, vr, okr, base);
            load_block(kr, vr, okr, base + 2 * BLK);
            process(kn2, vn2, okn, base + BLK);
        }
    }
    // Back to natural-log units for the merges (scores times the scale).
#pragma unroll
    for (int g = 0; g < G; ++g)
        if (m[g] != -INFINITY) m[g] *= scale;

    decode_merge<HD, G, LPR, 4>(m, l, o, s_m, s_l, s_o, [&](int g, int d, float M, float L, float acc) {
        const int h = kvh * G + g;
        const int64_t row = (int64_t)tok * H + h;
        if (ns > 1) {
            float* dst = part + (row * nsplit + split) * (HD + 2);
            dst[d] = acc;
            if (d == 0) {
                dst[HD] = M;
                dst[HD + 1] = L;
            }
            return;
        }
        if (sink) {
            const float sv = sink[h];
            const float mm = fmaxf(M, sv);
            const float a = M == -INFINITY ? 0.f : __expf(M - mm);
            L = L * a + __expf(sv - mm);
            acc *= a;
        }
        out[row * HD + d] = from_f32<T>(L > 0.f ? acc / L : 0.f);
    });
}

// Merge of split rows, one workgroup per (token, head) row, with the optional
// head sink folded in. Rows with a split count of 0 were written directly.
template <typename T>
__global__ __launch_bounds__(128) void paged_merge_kernel(const float* __restrict__ part,
                                                          T* __restrict__ out, int nsplit,
                                                          const int* __restrict__ nsplit_row,
                                                          int vhd, int H,
                                                          const float* __restrict__ sink) {
    const int64_t tok = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t r = tok * H + h;
    const int ns = min(nsplit, nsplit_row[r]);
    if (ns <= 0) return;
    const float* p = part + r * nsplit * (vhd + 2);
    if (ns <= kMergeFast && vhd <= 128) {
        // Every value a thread needs in one batch of loads (splits past the count
        // read zeros without an access), merged in registers.
        const uint32_t bytes = (uint32_t)(ns * (vhd + 2)) * 4u;
        const __amdgpu_buffer_rsrc_t rp = buffer_rsrc(p, bytes);
        const int d = min((int)threadIdx.x, vhd - 1);
        float mv[kMergeFast], lv[kMergeFast], ov[kMergeFast];
#pragma unroll
        for (int i = 0; i < kMergeFast; ++i) {
            const uint32_t row = (uint32_t)(i * (vhd + 2)) * 4u;
            const bool in = i < ns;
            mv[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rp, in ? row + vhd * 4u : bytes, 0, 0));
            lv[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rp, in ? row + vhd * 4u + 4u : bytes, 0, 0));
            ov[i] = __uint_as_float(
                __builtin_amdgcn_raw_buffer_load_b32(rp, in ? row + d * 4u : bytes, 0, 0));
        }
        float M = sink ? sink[h] : -INFINITY;
#pragma unroll
        for (int i = 0; i < kMergeFast; ++i)
            if (i < ns) M = fmaxf(M, mv[i]);
        float L = sink && M != -INFINITY ? __expf(sink[h] - M) : 0.f, acc = 0.f;
#pragma unroll
        for (int i = 0; i < kMergeFast; ++i) {
            const float w = i < ns && mv[i] != -INFINITY ? __expf(mv[i] - M) : 0.f;
            L = fmaf(w, lv[i], L);
            acc = fmaf(w, ov[i], acc);
        }
        if ((int)threadIdx.x < vhd)
            out[tok * ((int64_t)H * vhd) + (int64_t)h * vhd + threadIdx.x] =
                from_f32<T>(L > 0.f ? acc / L : 0.f);
        return;
    }
    float M = -INFINITY;
    for (int i = 0; i < ns; ++i) M = fmaxf(M, p[i * (vhd + 2) + vhd]);
    if (sink) M = fmaxf(M, sink[h]);
    float L = 0.f;
    for (int i = 0; i < ns; ++i) {
        const float m = p[i * (vhd + 2) + vhd];
        if (m != -INFINITY) L += p[i * (vhd + 2) + vhd + 1] * __expf(m - M);
    }
    if (sink) L += __expf(sink[h] - M);
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    T* o = out + tok * ((int64_t)H * vhd) + (int64_t)h * vhd;
    for (int d = threadIdx.x; d < vhd; d += blockDim.x) {
        float acc = 0.f;
        for (int i = 0; i < ns; ++i) {
            const float m = p[i * (vhd + 2) + vhd];
            if (m != -INFINITY) acc += p[i * (vhd + 2) + d] * __expf(m - M);
        }
        o[d] = from_f32<T>(acc * inv);
    }
}


__global__ void sink_to_f32_kernel(const void* src, int dtype, float* dst, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (dtype == ORTMI_F32) dst[i] = static_cast<const float*>(src)[i];
    else if (dtype == ORTMI_F16) dst[i] = (float)static_cast<const half_t*>(src)[i];
    else dst[i] = to_f32(static_cast<const uint16_t*>(src)[i]);
}

// ------------------------------------------------------ RotaryEmbedding --

template <typename T>
__global__ __launch_bounds__(256) void rotary_kernel(const T* __restrict__ x,
                                                     const int64_t* __restrict__ pos,
                                                     int pos_is_offset,
                                                     const T* __restrict__ cos_c,
                                                     const T* __restrict__ sin_c,
                                                     T* __restrict__ y, int B, int S, int NH,
                                                     int hd, int half, int bnsd,
                                                     int interleaved, int64_t total_pairs,
                                                     int64_t max_pos) {
    // One thread per (b, s, n, pair) plus pass-through of dims >= 2*half.
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int rot = 2 * half;
    const int per_head = half + (hd - rot);
    if (i >= total_pairs) return;
    const int64_t hidx = i / per_head;  // (b, s, n) flattened as b, s, n
    const int e = (int)(i % per_head);
    const int n = (int)(hidx % NH);
    const int64_t bs = hidx / NH;
    const int s = (int)(bs % S), b = (int)(bs / S);
    const int64_t base = bnsd ? (((int64_t)b * NH + n) * S + s) * hd
                              : ((int64_t)b * S + s) * (int64_t)NH * hd + (int64_t)n * hd;
    if (e >= half) {
        const int d = rot + (e - half);
        y[base + d] = x[base + d];
        return;
    }
    int64_t row;
    if (!pos) row = (int64_t)b * S + s;
    else if (pos_is_offset) row = pos[0] + s;
    else row = pos[(int64_t)b * S + s];
    // Out-of-range positions violate the op contract; clamp so reads stay in bounds.
    row = row < 0 ? 0 : (row >= max_pos ? max_pos - 1 : row);
    int ia, ib;
    rope_pair_index<T>(e, half, interleaved, ia, ib);
    const float c = to_f32(cos_c[row * half + e]), sn = to_f32(sin_c[row * half + e]);
    const float a = to_f32(x[base + ia]), bb = to_f32(x[base + ib]);
    y[base + ia] = from_f32<T>(a * c - bb * sn);
    y[base + ib] = from_f32<T>(bb * c + a * sn);
}

// ------------------------------------------------------------- helpers --

static size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

static int gqa_nsplit(int64_t BKV, int64_t nkeys, int& chunk, int per_cu = 2) {
    // One round of two workgroups per CU (the decode kernel's occupancy): longer
    // splits amortise the epilogue and the merge, and a second round would run
    // with a partial tail (B=8 KV=8 ctx 4097 on MI355X: 512 workgroups 66.5 us,
    // 1408 workgroups 73 us). Chunks are multiples of 64 keys. The copying
    // (growing) form takes two rounds (per_cu = 4): its stores and loads overlap
    // better over more, shorter splits (B=8 KV=8, 4096 past rows: 61.4 -> 59.2 us).
    const int64_t want = std::max<int64_t>(1, (int64_t)per_cu * device_cu_count() / BKV);
    int64_t c = (nkeys + want - 1) / want;
    c = ((c + 63) / 64) * 64;
    if (c < 64) c = 64;
    // The merge kernel weighs at most 1024 splits.
    const int64_t cmin = ((nkeys + 1023) / 1024 + 63) / 64 * 64;
    if (c < cmin) c = cmin;
    chunk = (int)c;
    return (int)((nkeys + c - 1) / c);
}

// Splits of a one-token step whose partials go to the o_proj GEMV: the GQA rule,
// with longer chunks when the partials of all heads would exceed what the GEMV
// stages (0 when even one split does not fit).
static int gqa_partials_nsplit(int64_t B, int64_t H, int64_t KV, int64_t hd, int64_t cap,
                               int& chunk) {
    const int64_t per_split = B * H * (hd + 2);
    const int64_t max_ns = kDecodeMergeMaxFloats / per_split;
    if (max_ns < 1) return 0;
    const int ns = gqa_nsplit(B * KV, cap, chunk);
    if (ns <= max_ns) return ns;
    int64_t c = (cap + max_ns - 1) / max_ns;
    c = (c + 63) / 64 * 64;
    chunk = (int)c;
    return (int)((cap + c - 1) / c);
}

}  // namespace ortmi

using namespace ortmi;

// ---------------------------------------------------------------- GQA API --

extern "C" size_t ortmi_group_query_attention_workspace_size(int64_t batch, int64_t seq_len,
                                                             int64_t num_heads, int64_t head_size,
                                                             int64_t total_kv) {
    // qrot (fp32-sized upper bound) + decode partials, or the prefill tiles' split
    // partials and per-row split counts.
    size_t q = align_up((size_t)batch * seq_len * num_heads * head_size * 4);
    // Chunks are at least 64 keys, so ceil(total_kv / 64) bounds the split count.
    const int64_t nkv = total_kv > 0 ? total_kv : 1;
    const int64_t ns = (nkv + 63) / 64;
    size_t part = align_up((size_t)batch * num_heads * (size_t)ns * (head_size + 2) * 4);
    if (seq_len > 1) {
        const size_t rows = (size_t)batch * seq_len * num_heads;
        part = std::max(part, align_up(rows * kPrefillSplits * (head_size + 2) * 4) +
                                  align_up(rows * 4));
    }
    // Head 96 takes the generic kernels for everything but the one-token decode.
    if (head_size == 96)
        return std::max(q + part, ortmi_group_query_attention_ex_workspace_size(
                                      batch, seq_len, num_heads, head_size));
    return q + part;
}

// Launch of the one-token decode kernel for G query heads per KV head. When the
// (batch x KV head x key split) grid is small, the G heads are spread over
// workgroups (each reading the same cached rows) so that fewer heads sit on one
// workgroup's critical path: a decode step at short context is bound by the
// instructions of one workgroup, not by bandwidth.
template <typename T, int HD>
static int launch_gqa_decode(int G, int B, int KV, int ns, int chunk, const T* q, const T* k,
                             const T* v, int64_t q_stride, int64_t kv_stride, const T* cos_c,
                             const T* sin_c, int half, int interleaved, const T* kpast,
                             const T* vpast, T* kpres, T* vpres, int64_t past_cap,
                             int64_t pres_cap, int copy_past, int vp, float sc, float* part,
                             T* out, const int* total_dev, int vp_max, hipStream_t st) {
    // One head per workgroup measured best at 20 workgroups (6 heads per KV head,
    // 640-row buffer): 7.3 us with the merge against 8.5 / 9.7 / 12.8 us for 2 / 3 / 6.
    // Spreading multiplies the K/V reads by G, so it is only taken when even the
    // spread grid fits one round.
    // The kernel addresses one (b, kv) slice of a cache with 32-bit byte offsets.
    const int64_t slice_rows = std::max(copy_past ? past_cap : (int64_t)0, pres_cap);
    ORTMI_REQUIRE(slice_rows * HD * (int64_t)sizeof(T) < (int64_t)UINT32_MAX,
                  "GroupQueryAttention decode: one (batch, kv head) slice of the KV cache "
                  "must be under 4 GiB");
    const int per = (int64_t)B * KV * ns * G <= 2L * device_cu_count() ? 1 : G;
    const int gsplit = G / per;
    dim3 grid((unsigned)(B * KV * gsplit), (unsigned)ns);
    auto launch = [&](auto gtag) {
        constexpr int GG = decltype(gtag)::value;
        hipLaunchKernelGGL((gqa_decode_kernel<T, HD, GG>), grid, dim3(256), 0, st, q, k, v,
                           q_stride, kv_stride, cos_c, sin_c, half, interleaved, kpast, vpast,
                           kpres, vpres, past_cap, pres_cap, copy_past, vp, chunk, ns, KV, sc,
                           part, out, total_dev, vp_max, gsplit);
    };
    switch (per) {  // query heads per workgroup
        case 1: launch(std::integral_constant<int, 1>()); break;
        case 2: launch(std::integral_constant<int, 2>()); break;
        case 3: launch(std::integral_constant<int, 3>()); break;
        case 4: launch(std::integral_constant<int, 4>()); break;
        case 5: launch(std::integral_constant<int, 5>()); break;
        case 6: launch(std::integral_constant<int, 6>()); break;
        case 7: launch(std::integral_constant<int, 7>()); break;
        default: launch(std::integral_constant<int, 8>()); break;
    }
    return check_launch("gqa_decode");
}

template <typename T, int HD>
static int run_gqa(const void* query, const void* key, const void* value, const void* past_key,
                   const void* past_value, int64_t cap, int total, const void* cos_c,
                   const void* sin_c, int half, void* output, void* pk, void* pv, int B, int S,
                   int H, int KV, float scale, int interleaved, void* ws, size_t ws_bytes,
                   hipStream_t st) {
    const int hd = HD;
    int vp = total - S;
    bool shared;
    if (vp < 0 || vp > cap) {
        shared = false;
        vp = (int)cap;
    } else {
        shared = cap > vp;
    }
    const int64_t pcap = shared ? cap : cap + S;
    const bool packed = key == nullptr;
    const int64_t q_stride = packed ? (int64_t)(H + 2 * KV) * hd : (int64_t)H * hd;
    const int64_t kv_stride = packed ? q_stride : (int64_t)KV * hd;
    const T* q = static_cast<const T*>(query);
    const T* k = packed ? q + (int64_t)H * hd : static_cast<const T*>(key);
    const T* v = packed ? q + (int64_t)(H + KV) * hd : static_cast<const T*>(value);
    const int nkeys = vp + S;
    const int G = H / KV;
    const float sc = scale != 0.f ? scale : 1.0f / sqrtf((float)hd);

    size_t need = ortmi_group_query_attention_workspace_size(B, S, H, hd, nkeys);
    if (!ws || ws_bytes < need)
        return fail(ORTMI_E_WORKSPACE, "GroupQueryAttention: workspace too small");
    T* qrot = static_cast<T*>(ws);
    float* part = reinterpret_cast<float*>(static_cast<char*>(ws) +
                                           align_up((size_t)B * S * H * hd * 4));

    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    const bool decode_fast = S == 1 && G >= 1 && G <= 8 &&
                             (!cos_c || interleaved || half % 8 == 0) && a16(q) && a16(k) &&
                             a16(v) && a16(pk) && a16(pv) && (cap == 0 || (a16(past_key) &&
                             a16(past_value)));
    // Past rows that must reach `present` when it is a different buffer: the fused
    // decode kernel copies them itself in the growing contract; otherwise a copy
    // kernel runs first (shared contract into a separate present copies all cap
    // rows; growing prefill copies the cap past rows).
    const bool aliased = (pk == past_key) && (pv == past_value);
    const bool fused_copy = decode_fast && !shared && !aliased;
    if (!aliased && !fused_copy && cap > 0) {
        const int vec_per_row = hd * (int)sizeof(T) / 16;
        const int64_t total_vec = (int64_t)B * KV * cap * vec_per_row;
        int grid = (int)std::min<int64_t>((total_vec + 255) / 256, 65536);
        hipLaunchKernelGGL(kv_copy_kernel, dim3(grid), dim3(256), 0, st,
                           static_cast<const uint4*>(past_key), static_cast<uint4*>(pk), cap,
                           pcap, cap, vec_per_row, total_vec);
        hipLaunchKernelGGL(kv_copy_kernel, dim3(grid), dim3(256), 0, st,
                           static_cast<const uint4*>(past_value), static_cast<uint4*>(pv), cap,
                           pcap, cap, vec_per_row, total_vec);
        if (int rc = check_launch("gqa kv copy")) return rc;
    }
    if (decode_fast) {
        // Splits over the cached rows; the new row falls to the last split (B=8 KV=8
        // with 4096 past rows: 8 splits of 512 instead of 7 of 576 and one of 65,
        // shared contract 35.0-36.0 -> 33.8-34.0 us).
        int chunk = 0;
        const int ns = gqa_nsplit((int64_t)B * KV, std::max(vp, 1), chunk, fused_copy ? 4 : 2);
        if (int rc = launch_gqa_decode<T, HD>(
                G, B, KV, ns, chunk, q, k, v, q_stride, kv_stride, static_cast<const T*>(cos_c),
                static_cast<const T*>(sin_c), half, interleaved, static_cast<const T*>(past_key),
                static_cast<const T*>(past_value), static_cast<T*>(pk), static_cast<T*>(pv), cap,
                pcap, fused_copy ? 1 : 0, vp, sc, part, static_cast<T*>(output), nullptr, 0, st))
            return rc;
        if (ns == 1) return ORTMI_OK;
        hipLaunchKernelGGL((attn_merge_kernel<T>), dim3(B * H), dim3(128), 0, st, part,
                           static_cast<T*>(output), ns, (const int*)nullptr, hd, H,
                           (int64_t)H * hd, (const int*)nullptr);
        return check_launch("gqa_merge");
    }
    hipLaunchKernelGGL((gqa_prep_kernel<T>), dim3(B * S, (H + KV + kPrepHeads - 1) / kPrepHeads),
                       dim3(64 * kPrepHeads), kPrepHeads * hd * sizeof(float), st,
                       q, k, v, static_cast<const T*>(cos_c), static_cast<const T*>(sin_c), half,
                       interleaved, qrot, static_cast<T*>(pk), static_cast<T*>(pv), B, S, H, KV,
                       hd, pcap, vp, q_stride, kv_stride);
    if (int rc = check_launch("gqa_prep")) return rc;
    const int QT = std::max(1, tile_rows_for<T>(HD, kGqaTileWaves) / G);
    const int tiles = (S + QT - 1) / QT;
    DenseKV dk{pk, pv, pcap, KV};
    // Key splits when the tiles alone leave CUs idle (a 512-token decoder prefill
    // has 50 tiles): about two workgroups per CU, chunks of at least 128 keys, at
    // most kPrefillSplits; the splits are merged per (token, head) row.
    int chunk = nkeys, ns = 1;
    {
        const int64_t wgs = (int64_t)B * tiles * KV;
        const int64_t want = std::min<int64_t>(
            kPrefillSplits, (2LL * device_cu_count() + wgs - 1) / std::max<int64_t>(wgs, 1));
        if (want > 1) {
            chunk = (int)std::max<int64_t>(128, ((nkeys + want - 1) / want + 63) / 64 * 64);
            ns = (nkeys + chunk - 1) / chunk;
        }
    }
    float* ppart = nullptr;
    int* prow = nullptr;
    if (ns > 1) {
        char* base = static_cast<char*>(ws) + align_up((size_t)B * S * H * hd * 4);
        ppart = reinterpret_cast<float*>(base);
        prow = reinterpret_cast<int*>(base + align_up((size_t)B * S * H * kPrefillSplits *
                                                      (hd + 2) * 4));
    }
    hipLaunchKernelGGL((gqa_tile_kernel<T, HD>), dim3(B * tiles, KV, ns),
                       dim3(tile_threads<T, HD, kGqaTileWaves>()), 0, st, qrot,
                       dk, S, QT, tiles, G, H, vp, sc, static_cast<T*>(output), chunk, ns, ppart,
                       prow);
    if (int rc = check_launch("gqa_tile")) return rc;
    if (ns == 1) return ORTMI_OK;
    hipLaunchKernelGGL((paged_merge_kernel<T>), dim3((unsigned)(B * S), (unsigned)H), dim3(128), 0,
                       st, ppart, static_cast<T*>(output), ns, prow, hd, H, (const float*)nullptr);
    return check_launch("gqa_tile_merge");
}

extern "C" int ortmi_group_query_attention(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, int32_t total_sequence_length, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, void* output, void* present_key,
    void* present_value, int64_t batch, int64_t seq_len, int64_t num_heads, int64_t kv_num_heads,
    int64_t head_size, float scale, int32_t rotary_interleaved, int32_t dtype, void* workspace,
    size_t workspace_bytes, void* stream) {
    // Claim/op contract of rust/src/ops/attention.rs:1527-1738 and 556-952.
    ORTMI_REQUIRE(num_heads > 0 && kv_num_heads > 0 && num_heads % kv_num_heads == 0,
                  "GroupQueryAttention: num_heads must be a positive multiple of kv_num_heads");
    ORTMI_REQUIRE(head_size == 64 || head_size == 96 || head_size == 128,
                  "GroupQueryAttention: head_size must be 64, 96 or 128");
    ORTMI_REQUIRE(batch > 0 && seq_len > 0 && past_cap >= 0, "GroupQueryAttention: bad shape");
    ORTMI_REQUIRE(query && output && present_key && present_value,
                  "GroupQueryAttention: null tensor");
    ORTMI_REQUIRE((key == nullptr) == (value == nullptr),
                  "GroupQueryAttention: key and value must both be given or both be packed");
    ORTMI_REQUIRE(past_cap == 0 || (past_key && past_value), "GroupQueryAttention: null past");
    ORTMI_REQUIRE(kv_num_heads <= 4096 && num_heads / kv_num_heads <= 64,
                  "GroupQueryAttention: too many heads per group");
    const bool rotary = cos_cache != nullptr;
    ORTMI_REQUIRE(rotary == (sin_cache != nullptr),
                  "GroupQueryAttention: cos_cache and sin_cache must both be given");
    int vp = total_sequence_length - (int)seq_len;
    if (vp < 0 || vp > past_cap) vp = (int)past_cap;
    if (rotary) {
        ORTMI_REQUIRE(rotary_half > 0 && 2 * rotary_half <= head_size,
                      "GroupQueryAttention: rotary dim exceeds head_size");
        ORTMI_REQUIRE(vp + seq_len <= max_pos,
                      "GroupQueryAttention: position exceeds the cos/sin cache");
    }
    if (past_cap > 0 && (past_key == present_key) != (past_value == present_value))
        return fail(ORTMI_E_INVALID, "GroupQueryAttention: present_key/value alias mismatch");
    const bool shared_c = (total_sequence_length - seq_len >= 0) &&
                          (total_sequence_length - seq_len <= past_cap) &&
                          past_cap > total_sequence_length - seq_len;
    if (!shared_c && past_cap > 0)
        ORTMI_REQUIRE(past_key != present_key,
                      "GroupQueryAttention: growing contract cannot write in place");
    if (shared_c)
        ORTMI_REQUIRE(total_sequence_length <= past_cap,
                      "GroupQueryAttention: total_sequence_length exceeds the KV buffer capacity");
    // Head 96 runs the one-token decode on the fast kernel (16-lane groups with 4
    // padding lanes); prompts, and decode steps the fast kernel does not take
    // (unaligned tensors, more than 8 query heads per KV head, a rotary half that is
    // not a multiple of 8), go to the generic kernels.
    if (head_size == 96) {
        const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
        const bool packed = key == nullptr;
        const void* kk = packed ? static_cast<const char*>(query) + num_heads * 96 * 2 : key;
        const void* vv = packed ? static_cast<const char*>(query) + (num_heads + kv_num_heads) * 96 * 2
                                : value;
        const bool fast = seq_len == 1 && num_heads / kv_num_heads <= 8 && dtype != ORTMI_F32 &&
                          (!rotary || rotary_interleaved || rotary_half % 8 == 0) && a16(query) &&
                          a16(kk) && a16(vv) && a16(present_key) && a16(present_value) &&
                          (past_cap == 0 || (a16(past_key) && a16(past_value)));
        if (!fast)
            return ortmi_group_query_attention_ex(
                query, key, value, past_key, past_value, past_cap, total_sequence_length,
                cos_cache, sin_cache, rotary_half, max_pos, nullptr, nullptr, 1e-6f, nullptr, 0, 0,
                0, 0, output, present_key, present_value, batch, seq_len, num_heads, kv_num_heads,
                head_size, scale, rotary_interleaved, dtype, workspace, workspace_bytes, stream);
    }
    hipStream_t st = as_stream(stream);
    const int B = (int)batch, S = (int)seq_len, H = (int)num_heads, KV = (int)kv_num_heads;
    const int half = (int)rotary_half;
#define ORTMI_GQA(T, HD)                                                                          \
    return run_gqa<T, HD>(query, key, value, past_key, past_value, past_cap,                      \
                          total_sequence_length, cos_cache, sin_cache, half, output, present_key, \
                          present_value, B, S, H, KV, scale, rotary_interleaved, workspace,       \
                          workspace_bytes, st)
    if (dtype == ORTMI_F16) {
        if (head_size == 64) ORTMI_GQA(half_t, 64);
        if (head_size == 96) ORTMI_GQA(half_t, 96);
        ORTMI_GQA(half_t, 128);
    }
    if (dtype == ORTMI_BF16) {
        if (head_size == 64) ORTMI_GQA(uint16_t, 64);
        if (head_size == 96) ORTMI_GQA(uint16_t, 96);
        ORTMI_GQA(uint16_t, 128);
    }
#undef ORTMI_GQA
    return fail(ORTMI_E_INVALID, "GroupQueryAttention: dtype must be fp16 or bf16");
}

// Capturable one-token decode step over a fixed-capacity shared KV buffer.
template <typename T, int HD>
static int run_gqa_decode_capturable(const void* query, const void* key, const void* value,
                                     void* kv_key, void* kv_value, int64_t cap,
                                     const int32_t* total_dev, const void* cos_c,
                                     const void* sin_c, int half, int64_t max_pos, void* output,
                                     int B, int H, int KV, float scale, int interleaved, void* ws,
                                     size_t ws_bytes, float* partials_out, hipStream_t st) {
    const int G = H / KV;
    const bool packed = key == nullptr;
    const int64_t q_stride = packed ? (int64_t)(H + 2 * KV) * HD : (int64_t)H * HD;
    const int64_t kv_stride = packed ? q_stride : (int64_t)KV * HD;
    const T* q = static_cast<const T*>(query);
    const T* k = packed ? q + (int64_t)H * HD : static_cast<const T*>(key);
    const T* v = packed ? q + (int64_t)(H + KV) * HD : static_cast<const T*>(value);
    const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (G < 1 || G > 8 || (cos_c && !interleaved && half % 8 != 0) || !a16(q) || !a16(k) ||
        !a16(v) || !a16(kv_key) || !a16(kv_value))
        return fail(ORTMI_E_INVALID, "GroupQueryAttention: form has no capturable decode kernel");
    float* part = partials_out;
    if (!part) {
        if (ws_bytes < ortmi_group_query_attention_workspace_size(B, 1, H, HD, cap) || !ws)
            return fail(ORTMI_E_WORKSPACE, "GroupQueryAttention: workspace too small");
        part = reinterpret_cast<float*>(static_cast<char*>(ws) + align_up((size_t)B * H * HD * 4));
    }
    // Splits are sized for a full buffer; splits past the live keys contribute
    // empty partials (max -inf, sum 0) that the merge weighs by zero.
    int chunk = 0;
    const int ns = partials_out ? gqa_partials_nsplit(B, H, KV, HD, cap, chunk)
                                : gqa_nsplit((int64_t)B * KV, cap, chunk);
    if (ns < 1) return fail(ORTMI_E_INVALID, "GroupQueryAttention: too many heads for partials");
    const float sc = scale != 0.f ? scale : 1.0f / sqrtf((float)HD);
    const int vp_max = (int)std::min<int64_t>(cap, cos_c ? max_pos : cap) - 1;
    if (int rc = launch_gqa_decode<T, HD>(
            G, B, KV, ns, chunk, q, k, v, q_stride, kv_stride, static_cast<const T*>(cos_c),
            static_cast<const T*>(sin_c), half, interleaved, static_cast<const T*>(kv_key),
            static_cast<const T*>(kv_value), static_cast<T*>(kv_key), static_cast<T*>(kv_value),
            cap, cap, 0, 0, sc, part, partials_out ? nullptr : static_cast<T*>(output), total_dev,
            vp_max, st))
        return rc;
    if (ns == 1 || partials_out) return ORTMI_OK;
    hipLaunchKernelGGL((attn_merge_kernel<T>), dim3(B * H), dim3(128), 0, st, part,
                       static_cast<T*>(output), ns, (const int*)nullptr, HD, H, (int64_t)H * HD,
                       (const int*)nullptr);
    return check_launch("gqa_merge");
}

static int gqa_decode_capturable_entry(
    const void* query, const void* key, const void* value, void* kv_key, void* kv_value,
    int64_t kv_cap, const int32_t* total_dev, const void* cos_cache, const void* sin_cache,
    int64_t rotary_half, int64_t max_pos, void* output, float* partials, int64_t batch,
    int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* workspace, size_t workspace_bytes,
    void* stream) {
    ORTMI_REQUIRE(num_heads > 0 && kv_num_heads > 0 && num_heads % kv_num_heads == 0,
                  "GroupQueryAttention: num_heads must be a positive multiple of kv_num_heads");
    ORTMI_REQUIRE(head_size == 64 || head_size == 96 || head_size == 128,
                  "GroupQueryAttention: head_size must be 64, 96 or 128");
    ORTMI_REQUIRE(batch > 0 && kv_cap > 0, "GroupQueryAttention: bad shape");
    ORTMI_REQUIRE(query && (output || partials) && kv_key && kv_value && total_dev,
                  "GroupQueryAttention: null tensor");
    ORTMI_REQUIRE((key == nullptr) == (value == nullptr),
                  "GroupQueryAttention: key and value must both be given or both be packed");
    const bool rotary = cos_cache != nullptr;
    ORTMI_REQUIRE(rotary == (sin_cache != nullptr),
                  "GroupQueryAttention: cos_cache and sin_cache must both be given");
    if (rotary)
        ORTMI_REQUIRE(rotary_half > 0 && 2 * rotary_half <= head_size && max_pos > 0,
                      "GroupQueryAttention: rotary dim exceeds head_size");
    hipStream_t st = as_stream(stream);
    const int B = (int)batch, H = (int)num_heads, KV = (int)kv_num_heads;
#define ORTMI_GQA_CAP(T, HD)                                                                   \
    return run_gqa_decode_capturable<T, HD>(query, key, value, kv_key, kv_value, kv_cap,       \
                                            total_dev, cos_cache, sin_cache, (int)rotary_half, \
                                            max_pos, output, B, H, KV, scale, rotary_interleaved, \
                                            workspace, workspace_bytes, partials, st)
    if (dtype == ORTMI_F16) {
        if (head_size == 64) ORTMI_GQA_CAP(half_t, 64);
        if (head_size == 96) ORTMI_GQA_CAP(half_t, 96);
        ORTMI_GQA_CAP(half_t, 128);
    }
    if (dtype == ORTMI_BF16) {
        if (head_size == 64) ORTMI_GQA_CAP(uint16_t, 64);
        if (head_size == 96) ORTMI_GQA_CAP(uint16_t, 96);
        ORTMI_GQA_CAP(uint16_t, 128);
    }
#undef ORTMI_GQA_CAP
    return fail(ORTMI_E_INVALID, "GroupQueryAttention: dtype must be fp16 or bf16");
}

extern "C" int ortmi_group_query_attention_decode_capturable(
    const void* query, const void* key, const void* value, void* kv_key, void* kv_value,
    int64_t kv_cap, const int32_t* total_sequence_length_device, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, void* output, int64_t batch,
    int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* workspace, size_t workspace_bytes,
    void* stream) {
    ORTMI_REQUIRE(output, "GroupQueryAttention: null output");
    return gqa_decode_capturable_entry(query, key, value, kv_key, kv_value, kv_cap,
                                       total_sequence_length_device, cos_cache, sin_cache,
                                       rotary_half, max_pos, output, nullptr, batch, num_heads,
                                       kv_num_heads, head_size, scale, rotary_interleaved, dtype,
                                       workspace, workspace_bytes, stream);
}

extern "C" int64_t ortmi_group_query_attention_decode_splits(int64_t batch, int64_t num_heads,
                                                             int64_t kv_num_heads,
                                                             int64_t head_size, int64_t kv_cap) {
    if (batch <= 0 || num_heads <= 0 || kv_num_heads <= 0 || head_size <= 0 || kv_cap <= 0)
        return 0;
    int chunk = 0;
    return gqa_partials_nsplit(batch, num_heads, kv_num_heads, head_size, kv_cap, chunk);
}

extern "C" int ortmi_group_query_attention_decode_partials(
    const void* query, const void* key, const void* value, void* kv_key, void* kv_value,
    int64_t kv_cap, const int32_t* total_sequence_length_device, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, float* partials, int64_t batch,
    int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* stream) {
    ORTMI_REQUIRE(partials, "GroupQueryAttention: null partials");
    return gqa_decode_capturable_entry(query, key, value, kv_key, kv_value, kv_cap,
                                       total_sequence_length_device, cos_cache, sin_cache,
                                       rotary_half, max_pos, nullptr, partials, batch, num_heads,
                                       kv_num_heads, head_size, scale, rotary_interleaved, dtype,
                                       nullptr, 0, stream);
}

// ------------------------------------- GQA without caller-owned workspace --

// Workspace of ortmi_group_query_attention_noalloc: device memory of this
// library, one copy per GPU, held until the process ends. Host code never passes
// `scratch` itself to a kernel (in host code the name is a host-side stand-in,
// not a device address); it uses the per-device address from
// hipGetSymbolAddress kept in g_scratch_addr.
constexpr size_t kGqaScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kGqaScratchBytes];

constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxScratchDevices];

// Device address of the current device's `scratch`, looked up once per device
// (with that device current) on the first call.
static int scratch_address(void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return check_launch("hipGetDevice");
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(ORTMI_E_INVALID, "GroupQueryAttention: device ordinal out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(ORTMI_E_HIP, std::string("GroupQueryAttention: hipGetSymbolAddress: ") +
                                         hipGetErrorString(e));
        }
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return ORTMI_OK;
}

extern "C" size_t ortmi_group_query_attention_noalloc_max_workspace(void) {
    return kGqaScratchBytes;
}

extern "C" int ortmi_group_query_attention_noalloc(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, int32_t total_sequence_length, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, void* output, void* present_key,
    void* present_value, int64_t batch, int64_t seq_len, int64_t num_heads, int64_t kv_num_heads,
    int64_t head_size, float scale, int32_t rotary_interleaved, int32_t dtype, void* stream) {
    ORTMI_REQUIRE(batch > 0 && seq_len > 0 && num_heads > 0 && head_size > 0 && past_cap >= 0,
                  "GroupQueryAttention: bad shape");
    int64_t vp = (int64_t)total_sequence_length - seq_len;
    if (vp < 0 || vp > past_cap) vp = past_cap;
    const size_t need =
        ortmi_group_query_attention_workspace_size(batch, seq_len, num_heads, head_size, vp + seq_len);
    if (need > kGqaScratchBytes)
        return fail(ORTMI_E_WORKSPACE,
                    "GroupQueryAttention (no-alloc): needs " + std::to_string(need) +
                        " bytes of workspace, above the library's fixed " +
                        std::to_string(kGqaScratchBytes) + "-byte scratch");
    void* ws = nullptr;
    if (int rc = scratch_address(&ws)) return rc;
    return ortmi_group_query_attention(query, key, value, past_key, past_value, past_cap,
                                       total_sequence_length, cos_cache, sin_cache, rotary_half,
                                       max_pos, output, present_key, present_value, batch, seq_len,
                                       num_heads, kv_num_heads, head_size, scale,
                                       rotary_interleaved, dtype, ws, kGqaScratchBytes, stream);
}

// ------------------------------------------------------- PagedAttention API --

static int paged_max_tiles(int64_t T, int64_t batch, int QT) {
    return (int)((T + QT - 1) / QT + batch);
}
static int paged_qt(int G) { return std::max(1, kTileRows / G); }
// Keys per split: at least 512, and at most 8 splits per row (bounds the partials).
static int paged_nsplit(int64_t max_context, int& chunk) {
    const int64_t c = std::max<int64_t>(512, ((max_context + 7) / 8 + 63) / 64 * 64);
    chunk = (int)c;
    return (int)std::max<int64_t>(1, (max_context + c - 1) / c);
}

extern "C" size_t ortmi_paged_attention_workspace_size(int64_t num_tokens, int64_t batch,
                                                       int64_t num_heads, int64_t kv_num_heads,
                                                       int64_t head_size, int64_t v_head_size,
                                                       int64_t max_context) {
    const int64_t vhd = v_head_size > 0 ? v_head_size : head_size;
    const int G = (int)(num_heads / (kv_num_heads > 0 ? kv_num_heads : 1));
    const int QT = paged_qt(G > 0 ? G : 1);
    const int mt = paged_max_tiles(num_tokens, batch, QT);
    int chunk;
    const int ns = paged_nsplit(max_context, chunk);
    const int64_t prow = num_tokens * num_heads;  // partial rows, token-major
    size_t sz = 0;
    sz += align_up((size_t)num_tokens * num_heads * head_size * 4);      // qrot
    sz += align_up((size_t)num_tokens * kv_num_heads * head_size * 4);   // knew
    sz += align_up((size_t)(mt + 1) * 16);                               // tiles + count
    sz += align_up((size_t)prow * 4);                                    // nsplit_row
    sz += align_up((size_t)prow * ns * (vhd + 2) * 4);                   // partials
    sz += align_up((size_t)num_heads * 4);                               // sink fp32
    return sz;
}

// PagedAttention for the forms the tile and decode kernels do not take: fp32, and
// head sizes (and LATENT value sizes) that are multiples of 16 up to 256 other
// than 64/128. The prep kernel writes RoPE'd/normalised queries and new keys to
// the workspace and the new rows to their cache slots; paged_generic_attn_kernel
// then gives each (token, head) row one workgroup of 16 teams x 16 lanes (the
// layout of the generic GroupQueryAttention kernel): keys [0, past) come from the
// cache through the block table, keys from past on from the new rows themselves
// (as attention.rs:2640-2700 concatenates them), causal, with the head_sink logit
// joining the softmax normaliser (attention.rs:2420-2450).
constexpr int kGenTeams = 16, kGenLanes = 16, kGenMaxPerLane = 16;
template <typename T>
__global__ __launch_bounds__(256) void paged_generic_attn_kernel(
    const T* __restrict__ qrot, const T* __restrict__ knew, const T* __restrict__ vnew,
    const T* __restrict__ kcache, const T* __restrict__ vcache, int64_t nslots, int blk,
    const int32_t* __restrict__ cum, const int32_t* __restrict__ past,
    const int32_t* __restrict__ bt, int batch, int maxb, const float* __restrict__ sink,
    T* __restrict__ out, int H, int KV, int hd, int vhd, float scale, int max_ctx) {
    __shared__ float s_m[kGenTeams], s_l[kGenTeams];
    __shared__ float s_acc[kGenTeams][kGenLanes * kGenMaxPerLane];
    const int row = blockIdx.x;  // tok * H + h
    const int h = row % H, tok = row / H;
    const int kvh = h / (H / KV);
    const int team = threadIdx.x / kGenLanes, lt = threadIdx.x % kGenLanes;
    const int E = hd / kGenLanes, EV = vhd / kGenLanes;
    int lo = 0, hi = batch;  // the sequence: last b with cum[b] <= tok
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (cum[mid] <= tok) lo = mid;
        else hi = mid;
    }
    // The sequence's token range clamped to [0, T), as the tile map clamps it, and
    // past to [0, max_ctx]: new key rows stay tokens of [0, T) and the walk stays
    // bounded whatever the control tensors hold. A token outside its sequence's
    // clamped range (a malformed cum_seqlens) belongs to no sequence: zero row.
    const int T_ = (int)(gridDim.x / H);
    const int b = lo;
    const int s0 = min(max(cum[b], 0), T_), s1 = min(max(cum[b + 1], s0), T_);
    const int pb = min(max(past[b], 0), max_ctx);
    T* orow = out + (int64_t)row * vhd;
    if (tok < s0 || tok >= s1) {
        for (int d = threadIdx.x; d < vhd; d += blockDim.x) orow[d] = from_f32<T>(0.f);
        return;
    }
    const int nk = min(pb + (tok - s0) + 1, max_ctx);  // causal: keys [0, past + i]
    // LATENT (vcache == nullptr): values are the first vhd dims of the key rows.
    const int64_t kslot = (int64_t)KV * hd, vslot = (int64_t)KV * vhd;
    const T* qrow = qrot + (int64_t)row * hd;
    float qv[kGenMaxPerLane], acc[kGenMaxPerLane];
#pragma unroll
    for (int e = 0; e < kGenMaxPerLane; ++e) {
        qv[e] = e < E ? to_f32(qrow[lt + kGenLanes * e]) : 0.f;
        acc[e] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int base = 0; base < nk; base += kGenTeams) {
        const int j = base + team;
        if (j >= nk) continue;  // uniform over the team's 16 lanes
        const T *kr, *vr;
        if (j < pb) {
            const int lb = j / blk;
            const int phys = lb < maxb ? bt[(int64_t)b * maxb + lb] : -1;
            const int64_t slot = phys < 0 ? -1 : (int64_t)phys * blk + j % blk;
            if (slot < 0 || slot >= nslots) continue;  // outside the cache: no key
            kr = kcache + slot * kslot + (int64_t)kvh * hd;
            vr = vcache ? vcache + slot * vslot + (int64_t)kvh * vhd : kr;
        } else {
            const int64_t t = s0 + (j - pb);
            kr = knew + t * kslot + (int64_t)kvh * hd;
            vr = vcache ? vnew + t * vslot + (int64_t)kvh * vhd : kr;
        }
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < kGenMaxPerLane; ++e)
            if (e < E) dot += qv[e] * to_f32(kr[lt + kGenLanes * e]);
        const float sc = group_sum<kGenLanes>(dot) * scale;
        const float mn = fmaxf(m, sc);
        const float corr = __expf(m - mn);  // m = -inf -> 0
        const float pe = __expf(sc - mn);
        l = l * corr + pe;
#pragma unroll
        for (int e = 0; e < kGenMaxPerLane; ++e)
            if (e < EV) acc[e] = acc[e] * corr + pe * to_f32(vr[lt + kGenLanes * e]);
        m = mn;
    }
    if (lt == 0) {
        s_m[team] = m;
        s_l[team] = l;
    }
#pragma unroll
    for (int e = 0; e < kGenMaxPerLane; ++e)
        if (e < EV) s_acc[team][lt + kGenLanes * e] = acc[e];
    __syncthreads();
    float M = -INFINITY;
    for (int tm = 0; tm < kGenTeams; ++tm) M = fmaxf(M, s_m[tm]);
    const float sk = sink ? sink[h] : -INFINITY;
    M = fmaxf(M, sk);
    for (int d = threadIdx.x; d < vhd; d += blockDim.x) {
        float num = 0.f, den = sink ? __expf(sk - M) : 0.f;
        for (int tm = 0; tm < kGenTeams; ++tm) {
            if (s_m[tm] == -INFINITY) continue;
            const float wt = __expf(s_m[tm] - M);
            num += wt * s_acc[tm][d];
            den += wt * s_l[tm];
        }
        orow[d] = from_f32<T>(num / den);
    }
}

template <typename T>
static int run_paged_generic(const void* query, const void* key, const void* value,
                             void* kcache, void* vcache, int64_t nblk, int blk,
                             const int32_t* cum, const int32_t* past, const int32_t* bt, int batch,
                             int maxb, int64_t T_, const void* cos_c, const void* sin_c, int half,
                             int64_t max_pos, int interleaved, int rot_off,
                             const int32_t* slot_mapping, const void* sink, int sink_dtype,
                             const void* qw, const void* kw, float eps, void* output, int H,
                             int KV, int hd, int vhd, float scale, int64_t max_context, void* ws,
                             hipStream_t st) {
    // The workspace layout of run_paged (qrot, knew, tile map, split counts, ...):
    // the prep kernel also builds the tile map, which nothing here reads.
    const int G = H / KV;
    const int QT = paged_qt(G);
    const int mt = paged_max_tiles(T_, batch, QT);
    char* p = static_cast<char*>(ws);
    T* qrot = reinterpret_cast<T*>(p);
    p += align_up((size_t)T_ * H * hd * 4);
    T* knew = reinterpret_cast<T*>(p);
    p += align_up((size_t)T_ * KV * hd * 4);
    int4* tiles = reinterpret_cast<int4*>(p);
    int* count = reinterpret_cast<int*>(tiles + mt);
    p += align_up((size_t)(mt + 1) * 16);
    int* nsplit_row = reinterpret_cast<int*>(p);
    p += align_up((size_t)T_ * H * 4);
    int chunk;
    const int ns = paged_nsplit(1, chunk);
    p += align_up((size_t)T_ * H * ns * (vhd + 2) * 4);
    float* sink32 = reinterpret_cast<float*>(p);
    const float sc = scale != 0.f ? scale : 1.0f / sqrtf((float)hd);
    if (T_ == 0) return ORTMI_OK;
    hipLaunchKernelGGL((paged_prep_kernel<T>),
                       dim3((unsigned)T_, (H + KV + kPrepHeads - 1) / kPrepHeads),
                       dim3(64 * kPrepHeads), kPrepHeads * hd * sizeof(float), st,
                       static_cast<const T*>(query), static_cast<const T*>(key),
                       static_cast<const T*>(value), static_cast<T*>(kcache),
                       static_cast<T*>(vcache), nblk, blk, cum, past, bt, batch, maxb,
                       static_cast<const T*>(cos_c), static_cast<const T*>(sin_c), half,
                       interleaved, rot_off, slot_mapping, static_cast<const T*>(qw),
                       static_cast<const T*>(kw), eps, H, KV, hd, vhd, qrot, knew, max_pos, QT,
                       mt, tiles, count, nsplit_row);
    if (int rc = check_launch("paged_prep")) return rc;
    if (sink) {
        hipLaunchKernelGGL(sink_to_f32_kernel, dim3((H + 63) / 64), dim3(64), 0, st, sink,
                           sink_dtype, sink32, H);
        if (int rc = check_launch("paged_sink")) return rc;
    }
    hipLaunchKernelGGL((paged_generic_attn_kernel<T>), dim3((unsigned)(T_ * H)), dim3(256), 0, st,
                       qrot, knew, static_cast<const T*>(value), static_cast<const T*>(kcache),
                       static_cast<const T*>(vcache), nblk * blk, blk, cum, past, bt, batch, maxb,
                       sink ? sink32 : nullptr, static_cast<T*>(output), H, KV, hd, vhd, sc,
                       (int)std::min<int64_t>(max_context, INT32_MAX));
    return check_launch("paged_generic_attn");
}

template <typename T, int HD, int VHD>
static int run_paged(const void* query, const void* key, const void* value, void* kcache,
                     void* vcache, int64_t nblk, int blk, const int32_t* cum, const int32_t* past,
                     const int32_t* bt, int batch, int maxb, int64_t T_, int64_t max_context,
                     const void* cos_c, const void* sin_c, int half, int64_t max_pos,
                     int interleaved, int rot_off, const int32_t* slot_mapping, const void* sink, int sink_dtype,
                     const void* qw, const void* kw, float eps, void* output, int H, int KV,
                     float scale, void* ws, size_t ws_bytes, hipStream_t st) {
    const int G = H / KV;
    // Tiles of the kernel used for T (the workspace is sized for the smaller tile,
    // which gives more tiles, so it bounds this layout too).
    const int QT = std::max(1, tile_rows_for<T>(VHD, kPagedTileWaves) / G);
    const int mt = paged_max_tiles(T_, batch, QT);
    int chunk;
    const int ns = paged_nsplit(max_context, chunk);
    const size_t need =
        ortmi_paged_attention_workspace_size(T_, batch, H, KV, HD, VHD, max_context);
    if (!ws || ws_bytes < need) return fail(ORTMI_E_WORKSPACE, "PagedAttention: workspace too small");
    char* p = static_cast<char*>(ws);
    T* qrot = reinterpret_cast<T*>(p);
    p += align_up((size_t)T_ * H * HD * 4);
    T* knew = reinterpret_cast<T*>(p);
    p += align_up((size_t)T_ * KV * HD * 4);
    int4* tiles = reinterpret_cast<int4*>(p);
    int* count = reinterpret_cast<int*>(tiles + mt);
    p += align_up((size_t)(mt + 1) * 16);
    const int64_t prow = T_ * H;
    int* nsplit_row = reinterpret_cast<int*>(p);
    p += align_up((size_t)prow * 4);
    float* part = reinterpret_cast<float*>(p);
    p += align_up((size_t)prow * ns * (VHD + 2) * 4);
    float* sink32 = reinterpret_cast<float*>(p);
    const float sc = scale != 0.f ? scale : 1.0f / sqrtf((float)HD);

    if (T_ > 0) {
        hipLaunchKernelGGL((paged_prep_kernel<T>),
                           dim3((unsigned)T_, (H + KV + kPrepHeads - 1) / kPrepHeads),
                           dim3(64 * kPrepHeads), kPrepHeads * HD * sizeof(float), st,
                           static_cast<const T*>(query),
                           static_cast<const T*>(key), static_cast<const T*>(value),
                           static_cast<T*>(kcache), static_cast<T*>(vcache), nblk, blk, cum, past,
                           bt, batch, maxb, static_cast<const T*>(cos_c),
                           static_cast<const T*>(sin_c), half, interleaved, rot_off, slot_mapping,
                           static_cast<const T*>(qw), static_cast<const T*>(kw), eps, H, KV, HD,
                           VHD, qrot, knew, max_pos, QT, mt, tiles, count, nsplit_row);
        if (int rc = check_launch("paged_prep")) return rc;
    }
    if (T_ == 0) return ORTMI_OK;
    if (sink) {
        hipLaunchKernelGGL(sink_to_f32_kernel, dim3((H + 63) / 64), dim3(64), 0, st, sink,
                           sink_dtype, sink32, H);
        if (int rc = check_launch("paged_sink")) return rc;
    }
    int blk_shift = 0;
    while ((1 << blk_shift) < blk && blk_shift < 30) ++blk_shift;
    const bool pow2 = (1 << blk_shift) == blk && blk_shift <= 12;
    PagedKV pk{kcache, vcache, knew, value, bt, nblk, blk, maxb, KV, pow2 ? blk_shift : -1,
               (int)std::min<int64_t>(max_context, INT32_MAX)};
    if (!vcache) pk.vnew = nullptr;
    // Single-token tiles go to the vector-unit decode kernel when the block size is a
    // power of two and values have the key's head size. It writes rows no
    // multi-token tile owns (output, partials, split counts) and runs before the
    // tile kernel on the same stream: beside it, on a second stream, its
    // workgroups took the CUs the tile workgroups (a whole CU each) were waiting
    // for, and the pair finished no sooner than in sequence.
    bool dec = false;
    if constexpr (VHD == HD) {
        dec = vcache && value && pow2 && (G == 1 || G == 2 || G == 4 || G == 8);
        auto launch = [&](auto kernel) {
            hipLaunchKernelGGL(kernel, dim3(mt, KV, ns), dim3(256), 0, st, tiles, count, cum,
                               past, pk, blk_shift, qrot, H, sc, sink ? sink32 : nullptr, chunk,
                               ns, static_cast<T*>(output), part, nsplit_row);
        };
        if (dec) {
            switch (G) {
                case 1: launch(paged_decode_kernel<T, HD, 1>); break;
                case 2: launch(paged_decode_kernel<T, HD, 2>); break;
                case 4: launch(paged_decode_kernel<T, HD, 4>); break;
                case 8: launch(paged_decode_kernel<T, HD, 8>); break;
                default: dec = false;
            }
            if (dec)
                if (int rc = check_launch("paged_decode")) return rc;
        }
    }
    const unsigned tile_wgs = (unsigned)(kXcds * (int64_t)mt * ((KV * ns + kXcds - 1) / kXcds));
    hipLaunchKernelGGL((paged_tile_kernel<T, HD, VHD>), dim3(tile_wgs),
                       dim3(tile_threads<T, VHD, kPagedTileWaves>()), 0, st, tiles,
                       count, cum, past, pk, qrot, G, H, sc, sink ? sink32 : nullptr, chunk, ns,
                       static_cast<T*>(output), part, nsplit_row, dec ? 1 : 0, mt);
    if (int rc = check_launch("paged_tile")) return rc;
    if (ns > 1) {
        hipLaunchKernelGGL((paged_merge_kernel<T>), dim3((unsigned)T_, (unsigned)H), dim3(128), 0, st, part,
                           static_cast<T*>(output), ns, nsplit_row, VHD, H,
                           sink ? sink32 : nullptr);
        return check_launch("paged_merge");
    }
    return ORTMI_OK;
}

extern "C" int ortmi_paged_attention(
    const void* query, const void* key, const void* value, void* key_cache, void* value_cache,
    int64_t num_blocks, int64_t block_size, const int32_t* cum_seqlens,
    const int32_t* past_seqlens, const int32_t* block_table, int64_t batch, int64_t max_blocks,
    int64_t num_tokens, int64_t max_context, const void* cos_cache, const void* sin_cache,
    int64_t rotary_half, int64_t rotary_max_pos, int32_t rotary_interleaved,
    int64_t rotary_offset,
    const int32_t* slot_mapping, const void* head_sink, const void* q_norm_weight,
    const void* k_norm_weight, float qk_norm_eps, void* output, int64_t num_heads,
    int64_t kv_num_heads, int64_t head_size, int64_t v_head_size, float scale, int32_t dtype,
    void* workspace, size_t workspace_bytes, void* stream) {
    // Claim/op contract of rust/src/ops/attention.rs:2746-2977 and 2495-2744.
    ORTMI_REQUIRE(num_heads > 0 && kv_num_heads > 0 && num_heads % kv_num_heads == 0,
                  "PagedAttention: bad num_heads/kv_num_heads");
    const int64_t vhd = v_head_size > 0 ? v_head_size : head_size;
    const bool latent = value_cache == nullptr;
    ORTMI_REQUIRE(latent == (value == nullptr),
                  "PagedAttention: value and value_cache must both be given (or both absent for LATENT)");
    ORTMI_REQUIRE(head_size > 0 && head_size % 16 == 0 && head_size <= 256,
                  "PagedAttention: head_size must be a multiple of 16 up to 256");
    ORTMI_REQUIRE(vhd == head_size || (latent && vhd % 16 == 0 && vhd <= head_size),
                  "PagedAttention: unsupported v_head_size");
    ORTMI_REQUIRE(batch > 0 && block_size > 0 && num_blocks > 0 && max_blocks > 0,
                  "PagedAttention: bad cache or batch shape");
    ORTMI_REQUIRE(num_tokens >= 0 && num_tokens < (1LL << 31), "PagedAttention: bad token count");
    ORTMI_REQUIRE(max_context > 0, "PagedAttention: max_context must be positive");
    ORTMI_REQUIRE(cum_seqlens && past_seqlens && block_table && key_cache && output,
                  "PagedAttention: null tensor");
    ORTMI_REQUIRE(num_tokens == 0 || (query && key), "PagedAttention: null query/key");
    ORTMI_REQUIRE((cos_cache != nullptr) == (sin_cache != nullptr),
                  "PagedAttention: cos_cache and sin_cache must both be given");
    ORTMI_REQUIRE(!cos_cache || (rotary_half > 0 && rotary_offset >= 0 &&
                                 rotary_offset + 2 * rotary_half <= head_size),
                  "PagedAttention: rotary dims exceed head_size");
    ORTMI_REQUIRE(!cos_cache || rotary_max_pos > 0, "PagedAttention: empty cos/sin cache");
    ORTMI_REQUIRE((q_norm_weight != nullptr) == (k_norm_weight != nullptr),
                  "PagedAttention: q/k norm weights must both be given");
    ORTMI_REQUIRE(num_heads / kv_num_heads <= 64, "PagedAttention: too many heads per group");
    hipStream_t st = as_stream(stream);
#define ORTMI_PA(T, HD, VHD)                                                                     \
    return run_paged<T, HD, VHD>(query, key, value, key_cache, value_cache, num_blocks,          \
                                 (int)block_size, cum_seqlens, past_seqlens, block_table,        \
                                 (int)batch, (int)max_blocks, num_tokens, max_context,           \
                                 cos_cache, sin_cache, (int)rotary_half, rotary_max_pos,         \
                                 rotary_interleaved,                                             \
                                 (int)rotary_offset, slot_mapping, head_sink, dtype,             \
                                 q_norm_weight, k_norm_weight, qk_norm_eps, output,              \
                                 (int)num_heads, (int)kv_num_heads, scale, workspace,            \
                                 workspace_bytes, st)
    // fp32 and the head sizes the tile/decode kernels do not take run the generic kernels.
    const bool fused = dtype != ORTMI_F32 && (head_size == 64 || head_size == 128) &&
                       (vhd == head_size || vhd == 64) && rotary_offset % 8 == 0;
    if (!fused) {
        const size_t need = ortmi_paged_attention_workspace_size(
            num_tokens, batch, num_heads, kv_num_heads, head_size, v_head_size, max_context);
        if (!workspace || workspace_bytes < need)
            return fail(ORTMI_E_WORKSPACE, "PagedAttention: workspace too small");
#define ORTMI_PAG(T)                                                                              \
    return run_paged_generic<T>(query, key, value, key_cache, value_cache, num_blocks,            \
                                (int)block_size, cum_seqlens, past_seqlens, block_table,          \
                                (int)batch, (int)max_blocks, num_tokens, cos_cache, sin_cache,    \
                                (int)rotary_half, rotary_max_pos, rotary_interleaved,             \
                                (int)rotary_offset, slot_mapping, head_sink, dtype,               \
                                q_norm_weight, k_norm_weight, qk_norm_eps, output,                \
                                (int)num_heads, (int)kv_num_heads, (int)head_size, (int)vhd,      \
                                scale, max_context, workspace, st)
        if (dtype == ORTMI_F32) ORTMI_PAG(float);
        if (dtype == ORTMI_F16) ORTMI_PAG(half_t);
        if (dtype == ORTMI_BF16) ORTMI_PAG(uint16_t);
#undef ORTMI_PAG
        return fail(ORTMI_E_INVALID, "PagedAttention: dtype must be fp32, fp16 or bf16");
    }
    if (dtype == ORTMI_F16) {
        if (head_size == 64) ORTMI_PA(half_t, 64, 64);
        if (vhd == 64) ORTMI_PA(half_t, 128, 64);
        ORTMI_PA(half_t, 128, 128);
    }
    if (dtype == ORTMI_BF16) {
        if (head_size == 64) ORTMI_PA(uint16_t, 64, 64);
        if (vhd == 64) ORTMI_PA(uint16_t, 128, 64);
        ORTMI_PA(uint16_t, 128, 128);
    }
#undef ORTMI_PA
    return fail(ORTMI_E_INVALID, "PagedAttention: dtype must be fp32, fp16 or bf16");
}

// ------------------------------------------------------- RotaryEmbedding --

extern "C" int ortmi_rotary_embedding(const void* x, const int64_t* position_ids,
                                      int32_t pos_is_offset, const void* cos_cache,
                                      const void* sin_cache, int64_t max_pos, void* y,
                                      int64_t batch,
                                      int64_t seq_len, int64_t num_heads, int64_t head_size,
                                      int64_t rotary_half, int32_t is_bnsd, int32_t interleaved,
                                      int32_t dtype, void* stream) {
    ORTMI_REQUIRE(x && y && cos_cache && sin_cache, "RotaryEmbedding: null tensor");
    ORTMI_REQUIRE(batch >= 0 && seq_len >= 0 && num_heads > 0 && head_size > 0,
                  "RotaryEmbedding: bad shape");
    ORTMI_REQUIRE(rotary_half > 0 && 2 * rotary_half <= head_size,
                  "RotaryEmbedding: rotary dim exceeds head_size");
    ORTMI_REQUIRE(max_pos > 0, "RotaryEmbedding: empty cos/sin cache");
    ORTMI_REQUIRE(position_ids || max_pos >= batch * seq_len,
                  "RotaryEmbedding: per-token cos/sin must have batch*seq_len rows");
    const int64_t per_head = rotary_half + (head_size - 2 * rotary_half);
    const int64_t total = batch * seq_len * num_heads * per_head;
    if (total == 0) return ORTMI_OK;
    const int grid = (int)((total + 255) / 256);
    hipStream_t st = as_stream(stream);
#define ORTMI_ROPE(T)                                                                             \
    hipLaunchKernelGGL((rotary_kernel<T>), dim3(grid), dim3(256), 0, st, static_cast<const T*>(x), \
                       position_ids, pos_is_offset, static_cast<const T*>(cos_cache),            \
                       static_cast<const T*>(sin_cache), static_cast<T*>(y), (int)batch,         \
                       (int)seq_len, (int)num_heads, (int)head_size, (int)rotary_half, is_bnsd,  \
                       interleaved, total, max_pos);                                             \
    return check_launch("rotary")
    if (dtype == ORTMI_F32) { ORTMI_ROPE(float); }
    if (dtype == ORTMI_F16) { ORTMI_ROPE(half_t); }
    if (dtype == ORTMI_BF16) { ORTMI_ROPE(uint16_t); }
#undef ORTMI_ROPE
    return fail(ORTMI_E_INVALID, "RotaryEmbedding: unsupported dtype");
}
