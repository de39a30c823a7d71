// Int4 decoder decode step as one persistent kernel ("decode program") for gfx950.
//
// One cooperative launch runs a whole one-token step of a Llama-style int4
// decoder: embedding row -> per layer [(Skip)SimplifiedLayerNorm, merged QKV
// MatMulNBits, GroupQueryAttention over the shared KV cache with in-op RoPE,
// o_proj MatMulNBits, SkipSimplifiedLayerNorm, gate/up MatMulNBits with SwiGLU,
// down MatMulNBits] -> final SkipSimplifiedLayerNorm -> lm_head MatMulNBits ->
// greedy argmax. The reference reaches the same one-dispatch-per-token shape with
// a shapeless mlx_compile trace of the decode graph (rust/src/compiled.rs:1-28,
// 503-822); here the step is a fixed program of phases separated by grid-wide
// barriers.
//
// Why one kernel: at batch 1 every MatMulNBits of this decoder moves 1.3-16 MB,
// which the GPU streams in 1-3 us, while a dependent kernel boundary costs about
// 1.5 us and each small kernel spends another 1-2 us filling and draining. Here
// the weights of the next phase do not depend on the activations, so every wave
// issues the loads of its share of the next phase's weights into registers
// before it waits at the barrier: the HBM latency hides behind the
// synchronisation.
//
// Grid: one 512-thread workgroup per CU (co-resident by the cooperative launch).
// Wave 0 of each workgroup synchronises the grid; waves 1..7 do the row work, so
// their outstanding weight loads never stall the barrier's polling loads (loads
// and stores share one in-order counter per wave on this architecture).
//
// Cross-workgroup data: phase outputs are written with device-coherent (sc1)
// stores and read with sc1 loads; a barrier is entered after the wave's stores
// completed. Barrier: per-XCD arrival counters (workgroup i is on XCD i % 8),
// the last arrival of an XCD bumps a top counter that every workgroup polls.
// Every spin is bounded (50 ms of the 100 MHz realtime clock): a workgroup that
// times out raises the abort word, every other workgroup leaves at its next poll,
// and the launch reports status 1. Counters come in two sets used by alternate
// launches: a launch zeroes the other set after its first barrier, so the next
// launch starts from zero without any host work.
//
// Rounding follows the unfused ops of the fp16 graph: residual sums and
// normalised activations, MatMulNBits outputs, the RoPE'd query/key and the
// attention output are rounded to fp16 where the graph stores them; sums and
// softmax state are fp32.
#include "common.h"

namespace ortmi {
namespace dprog {

constexpr int kThreads = 512;
constexpr int kComputeWaves = 7;      // waves 1..7
constexpr int kSC1 = 16;              // buffer cache policy: device-coherent (sc1)
constexpr int kGMax = 8;              // query heads per KV head
constexpr int kNSMax = 8;             // key splits per KV head
constexpr int kKeySlots = kComputeWaves * 4;  // key rows per attention step
constexpr int kPrefSteps = 4;         // attention steps whose K/V rows are prefetched
constexpr int kIChunksPerLane = 5;    // down_proj: K = I <= 5 * 64 * 32 = 10240
constexpr unsigned long long kSpinTicks = 5000000ull;  // 50 ms

// Control block (uint32 words, one 128-byte line per counter).
constexpr int kCtlParity = 0;
constexpr int kCtlAbort = 32;
__host__ __device__ constexpr int ctl_top(int set) { return 32 * (2 + 9 * set); }
__host__ __device__ constexpr int ctl_xcd(int set, int x) { return 32 * (3 + 9 * set + x); }
constexpr size_t kCtlBytes = 4096;

struct Params {
    const OrtmiDecoderLayer* layers;
    int L, D, H, KV, I, V, cap, max_pos, half, nwg;
    float scale, final_eps;
    const half_t* embed;
    int64_t embed_rows;
    const int64_t* input_id;
    const int32_t* total;
    const half_t* cos;
    const half_t* sin;
    const half_t* final_gamma;
    const uint8_t* lm_w;
    const half_t* lm_s;
    half_t* logits;
    int64_t* next_id;
    int32_t* status;
    uint32_t* ctl;
    half_t* qkv;
    float* part;
    half_t* y;
    half_t* act;
    half_t* dout;
    float4* argp;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)bytes, kBufferWord3);
}
template <int POL>
__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <int POL>
__device__ __forceinline__ void st128(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
    u32x4_t t = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(t, r, off, 0, POL);
}
__device__ __forceinline__ unsigned atomic_add_dev(uint32_t* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned load_dev(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_dev(uint32_t* p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_status(int32_t* s, int v) {
    if (s) __hip_atomic_store(s, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float h2f(uint32_t bits16) {
    return (float)__builtin_bit_cast(half_t, (uint16_t)bits16);
}
__device__ __forceinline__ uint32_t f2h(float x) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (half_t)x);
}
__device__ __forceinline__ float r16(float x) { return (float)(half_t)x; }

// Grid barrier, called by every thread of every workgroup; wave 0 lane 0 arrives
// and polls once every wave's stores of the phase have completed.
struct Barrier {
    uint32_t* ctl;
    int set;
    unsigned round;
};
__device__ __forceinline__ bool grid_sync(Barrier& b, int nwg, int* s_flag, int32_t* status) {
    // Compute waves have waited for their stores before issuing the next phase's
    // prefetch (which must stay in flight across the barrier); the sync wave has
    // nothing in flight but its own staging stores.
    if (threadIdx.x < 64) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    ++b.round;
    if (threadIdx.x == 0) {
        const int x = blockIdx.x % kXcds;
        const unsigned per = (unsigned)(nwg / kXcds);
        const unsigned prev = atomic_add_dev(b.ctl + ctl_xcd(b.set, x), 1u);
        if (prev + 1 == b.round * per) atomic_add_dev(b.ctl + ctl_top(b.set), 1u);
        const unsigned target = b.round * (unsigned)kXcds;
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        int ok = 1;
        for (unsigned it = 0;; ++it) {
            if ((int)(load_dev(b.ctl + ctl_top(b.set)) - target) >= 0) break;
            if ((it & 15) == 15 && load_dev(b.ctl + kCtlAbort) != 0) {
                ok = 0;
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
                store_dev(b.ctl + kCtlAbort, 1u);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!ok) store_status(status, 1);
        *s_flag = ok;
    }
    __syncthreads();
    return *s_flag != 0;
}

// 16 lanes (dims 8*li .. 8*li+7 of one head) rotate their 8 values, non-interleaved
// pairs (i, i + half) over dims [0, 2*half); the partner lane is li ^ (half / 8)
// inside the same 16-lane group (half is a multiple of 8 and at most 64).
__device__ __forceinline__ void rope8(float (&x)[8], int li, int half, const half_t* cs,
                                      const half_t* sn) {
    if (half == 0) return;
    const int off = half / 8;
    const int lane = threadIdx.x & 63;
    const int partner = (lane & ~15) | ((li < off || (li >= 2 * off)) ? li + off : li - off);
    float px[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) px[i] = __shfl(x[i], partner & 63, 64);
    const int d0 = li * 8;
    if (d0 >= 2 * half) return;
    const bool low = d0 < half;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int p = (low ? d0 : d0 - half) + i;
        const float c = (float)cs[p], s = (float)sn[p];
        x[i] = low ? x[i] * c - px[i] * s : x[i] * c + px[i] * s;
    }
}

// ------------------------------------------------------------ weight rows
// Row chunks of one phase are fetched straight into LDS (buffer_load_dwordx4
// ... lds: lane i's 16 bytes land at the slot base + 16 * i), so the weights a
// wave prefetches across a barrier hold no registers. A compute wave owns
// kRegionSlots slots of 64 x 16 bytes; the per-chunk fp16 scales stay in VGPRs.
// Chunk c = li + j * LPR of row n goes to slot `slot0 + j`; rows past N and
// chunks past C read zeros (offsets past the buffer ranges), so the loads are
// unconditional.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint4* slot) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        r, (__attribute__((address_space(3))) void*)slot, 16, voff, 0, 0, kCachePolicyNT);
}

struct WeightRef {
    __amdgpu_buffer_rsrc_t w, s;
    uint32_t w_end, s_end;
    int N, C;
};
__device__ __forceinline__ WeightRef weight_ref(const uint8_t* w, const void* s, int N, int C) {
    WeightRef r;
    r.w_end = (uint32_t)N * (uint32_t)C * 16u;
    r.s_end = (uint32_t)N * (uint32_t)C * 2u;
    r.w = rsrc(w, r.w_end);
    r.s = rsrc(s, r.s_end);
    r.N = N;
    r.C = C;
    return r;
}

template <int LPR, int CPL>
__device__ __forceinline__ void fetch_rows(const WeightRef& wr, int n, int li, uint4* slot0,
                                           uint32_t (&sc)[CPL]) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        const bool ok = n < wr.N && c < wr.C;
        dma16(wr.w, ok ? (uint32_t)n * (uint32_t)(16 * wr.C) + 16u * c : wr.w_end, slot0 + j * 64);
        sc[j] = __builtin_amdgcn_raw_buffer_load_b16(
            wr.s, ok ? ((uint32_t)n * (uint32_t)wr.C + c) * 2u : wr.s_end, 0, 0);
    }
}

// Dot product of a lane's chunks (in LDS slots) with the staged activations (pair
// order, 4 uint4 per 32-code chunk), symmetric int4 (zero point 8):
// sum_j s_j * sum(a * (q - 8)).
template <int LPR, int CPL>
__device__ __forceinline__ float row_dot(const uint4* slot0, const uint32_t (&sc)[CPL],
                                         const uint4* sA, int C, int li) {
    const half_t zo = (half_t)1032.0f;
    const half2_t zoff = {zo, zo};
    const int lane = threadIdx.x & 63;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        if (c < C) {
            const uint4 av[4] = {sA[4 * c], sA[4 * c + 1], sA[4 * c + 2], sA[4 * c + 3]};
            acc = fmaf(h2f(sc[j]), dot32_pairs(av, slot0[j * 64 + lane], zoff), acc);
        }
    }
    return acc;
}

// Register form for the lm_head stream (after the layer loop, where registers
// are free): the chunks themselves in VGPRs.
template <int CPL>
struct Rows {
    uint4 w[CPL];
    uint32_t s[CPL];
};
template <int LPR, int CPL>
__device__ __forceinline__ void load_rows(Rows<CPL>& r, const WeightRef& wr, int n, int li) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        const bool ok = n < wr.N && c < wr.C;
        r.w[j] = ld128<kCachePolicyNT>(
            wr.w, ok ? (uint32_t)n * (uint32_t)(16 * wr.C) + 16u * c : wr.w_end);
        r.s[j] = __builtin_amdgcn_raw_buffer_load_b16(
            wr.s, ok ? ((uint32_t)n * (uint32_t)wr.C + c) * 2u : wr.s_end, 0, 0);
    }
}
template <int LPR, int CPL>
__device__ __forceinline__ float rows_dot(const Rows<CPL>& r, const uint4* sA, int C, int li) {
    const half_t zo = (half_t)1032.0f;
    const half2_t zoff = {zo, zo};
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        if (c < C) {
            const uint4 av[4] = {sA[4 * c], sA[4 * c + 1], sA[4 * c + 2], sA[4 * c + 3]};
            acc = fmaf(h2f(r.s[j]), dot32_pairs(av, r.w[j], zoff), acc);
        }
    }
    return acc;
}

// Residual add + RMS norm of one D-vector into LDS: r = fp16(in + r_prev) (or
// r = in when r_prev is not added), a = fp16(r * rsqrt(mean(r^2) + eps) * gamma),
// r kept in sR, a staged in pair order in sA. `in` comes from `src` through sc1
// loads (or plain loads for a constant table).
template <int POL>
__device__ __forceinline__ void norm_stage(const half_t* src, bool add_prev,
                                           const half_t* gamma, float eps, int D, uint4* sR,
                                           uint4* sA, float* sRed) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int units = D / 8;
    const __amdgpu_buffer_rsrc_t rs = rsrc(src, (uint32_t)D * 2);
    float ss = 0.f;
    for (int u = tid; u < units; u += kThreads) {
        uint4 v = ld128<POL>(rs, (uint32_t)u * 16);
        if (add_prev) {
            const uint4 pv = sR[u];
            const half_t* a = reinterpret_cast<const half_t*>(&v);
            const half_t* b = reinterpret_cast<const half_t*>(&pv);
            half_t t[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) t[e] = (half_t)((float)a[e] + (float)b[e]);
            v = *reinterpret_cast<const uint4*>(t);
        }
        sR[u] = v;
        const half_t* t = reinterpret_cast<const half_t*>(&v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)t[e] * (float)t[e];
    }
    ss = wave_sum(ss);
    if (lane == 0) sRed[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) tot += sRed[w];
    const float scale = 1.0f / sqrtf(tot / (float)D + eps);
    for (int u = tid; u < units; u += kThreads) {
        const uint4 v = sR[u];
        const uint4 gv = reinterpret_cast<const uint4*>(gamma)[u];
        const half_t* t = reinterpret_cast<const half_t*>(&v);
        const half_t* g = reinterpret_cast<const half_t*>(&gv);
        half_t o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (half_t)((float)t[e] * scale * (float)g[e]);
        sA[u] = permute_act8(*reinterpret_cast<const uint4*>(o));
    }
    __syncthreads();
}

// Copy n fp16 values written by other workgroups (sc1) into LDS in pair order.
__device__ __forceinline__ void stage_vec(const half_t* src, int n, uint4* sA) {
    const __amdgpu_buffer_rsrc_t rs = rsrc(src, (uint32_t)n * 2);
    for (int u = threadIdx.x; u < n / 8; u += kThreads)
        sA[u] = permute_act8(ld128<kSC1>(rs, (uint32_t)u * 16));
    __syncthreads();
}

__device__ __forceinline__ void st_half_sc1(half_t* base, uint32_t bytes, int idx, float v) {
    __builtin_amdgcn_raw_buffer_store_b16((uint16_t)f2h(v), rsrc(base, bytes), (uint32_t)idx * 2u,
                                          0, kSC1);
}

// Online-softmax state of a lane (8 dims) for N query heads.
template <int N>
struct AttnState {
    float m[N], l[N], o[N][8];
};

constexpr int gu_groups(int cpld) { return cpld == 3 ? 3 : 2; }
// Slot plan of a compute wave's LDS region (chunks of 64 x 16 bytes):
//   QKV [0, CPLD)              prefetched at the end of phase E (or at start)
//   attention K [0, P), V [P, 2P), P = kPrefSteps   end of phase A
//   o_proj [GU, GU + CPLD)      end of phase A      (GU = gate/up slots)
//   gate/up [0, GU)             end of phase B
//   down [GU, GU + 5)           end of phase C
// Every range is written only after the data it overlaps was consumed.
constexpr int region_slots(int cpld) {
    const int gu = gu_groups(cpld) * cpld;
    const int att = 2 * kPrefSteps;
    const int lo = gu > att ? gu : att;
    return lo + (cpld > kIChunksPerLane ? cpld : kIChunksPerLane);
}

template <int HD, int CPLD, int G>
__global__ __launch_bounds__(kThreads, 1) void decode_program_kernel(Params p) {
    extern __shared__ uint4 smem[];
    __shared__ float sRed[16];
    __shared__ int s_flag;
    __shared__ float s_am[kComputeWaves][kGMax], s_al[kComputeWaves][kGMax];
    __shared__ float s_arg_v[8];
    __shared__ int s_arg_i[8];
    constexpr int kGu = gu_groups(CPLD);
    constexpr int kGuSlots = kGu * CPLD;
    constexpr int kSlotsLo = kGuSlots > 2 * kPrefSteps ? kGuSlots : 2 * kPrefSteps;
    constexpr int kRegion = region_slots(CPLD);
    static_assert(kSlotsLo + CPLD <= kRegion && kSlotsLo + kIChunksPerLane <= kRegion, "slots");

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wg = blockIdx.x, nwg = p.nwg;
    const int cw = wave - 1;  // compute wave index, -1 for the sync wave
    const int TW = kComputeWaves * nwg;
    const int gw = cw * nwg + wg;  // global compute-wave index (spreads work over CUs)
    const int D = p.D, H = p.H, KV = p.KV, I = p.I;
    const int NQ = (H + 2 * KV) * HD;
    const int CD = D / 32, CO = H * HD / 32, CI = I / 32;
    const int li16 = lane & 15, grp = lane >> 4;

    // LDS: weight regions (7 waves), activations / attention merge area, residual.
    uint4* sW = smem;
    uint4* wreg = sW + (size_t)(cw < 0 ? 0 : cw) * kRegion * 64;
    uint4* sA = sW + (size_t)kComputeWaves * kRegion * 64;
    float* sO = reinterpret_cast<float*>(sA);  // [7][kGMax][HD], phase B only
    const int a_units = (I > D ? I : D) / 8;
    const int o_units = kComputeWaves * kGMax * HD / 4;
    uint4* sR = sA + (a_units > o_units ? a_units : o_units);

    // Total length, context, splits: the same on every workgroup.
    const int total = *p.total;
    if (total < 1 || total > p.cap || (p.half > 0 && total > p.max_pos)) {
        if (wg == 0 && tid == 0) store_status(p.status, 3);
        return;
    }
    const int ctx = total - 1;  // cached keys; the new key sits at index ctx
    int NS = (total + kKeySlots * kPrefSteps - 1) / (kKeySlots * kPrefSteps);
    NS = NS < 1 ? 1 : (NS > kNSMax ? kNSMax : NS);
    const int split_keys = (total + NS - 1) / NS;

    Barrier bar{p.ctl, 0, 0};
    bar.set = (int)load_dev(p.ctl + kCtlParity) & 1;

    // Token id and embedding row (negative ids count from the end).
    int64_t id = *p.input_id;
    if (id < 0) id += p.embed_rows;
    const bool bad_id = id < 0 || id >= p.embed_rows;
    if (bad_id) id = 0;

    // Attention work of this workgroup: KV head a_kvh, keys [k0, k1).
    const bool attn_wg = wg < KV * NS;
    const int a_kvh = wg / NS, a_split = wg % NS;
    const int k0 = a_split * split_keys;
    const int k1 = min(k0 + split_keys, total);
    const int slot = (cw < 0 ? 0 : cw) * 4 + grp;

    uint32_t sq[CPLD], so[CPLD], sg[kGu][CPLD], sd[kIChunksPerLane];

    auto qkv_fetch = [&](const OrtmiDecoderLayer& ly) {
        const WeightRef wr = weight_ref(ly.qkv_weight, ly.qkv_scales, NQ, CD);
        const int ng = (NQ + 3) / 4;
        fetch_rows<16, CPLD>(wr, gw < ng ? 4 * gw + grp : NQ, li16, wreg, sq);
    };
    auto kv_fetch = [&](const OrtmiDecoderLayer& ly) {
        const uint32_t bytes = (uint32_t)KV * p.cap * HD * 2;
        const __amdgpu_buffer_rsrc_t rk = rsrc(ly.k_cache, bytes), rv = rsrc(ly.v_cache, bytes);
#pragma unroll
        for (int t = 0; t < kPrefSteps; ++t) {
            const int key = k0 + t * kKeySlots + slot;
            const bool ok = attn_wg && key < k1 && key < ctx;
            const uint32_t off = ok ? ((uint32_t)(a_kvh * p.cap + key) * HD + li16 * 8) * 2u : bytes;
            dma16(rk, off, wreg + t * 64);
            dma16(rv, off, wreg + (kPrefSteps + t) * 64);
        }
    };
    auto o_fetch = [&](const OrtmiDecoderLayer& ly) {
        const WeightRef wr = weight_ref(ly.o_weight, ly.o_scales, D, CO);
        const int ng = (D + 3) / 4;
        fetch_rows<16, CPLD>(wr, gw < ng ? 4 * gw + grp : D, li16, wreg + kSlotsLo * 64, so);
    };
    auto gu_fetch = [&](const OrtmiDecoderLayer& ly) {
        const WeightRef wr = weight_ref(ly.gate_up_weight, ly.gate_up_scales, 2 * I, CD);
        const int ng = (2 * I + 3) / 4;
#pragma unroll
        for (int k = 0; k < kGu; ++k) {
            const int g = gw + k * TW;
            fetch_rows<16, CPLD>(wr, g < ng ? 4 * g + grp : 2 * I, li16, wreg + k * CPLD * 64,
                                 sg[k]);
        }
    };
    auto down_fetch = [&](const OrtmiDecoderLayer& ly) {
        const WeightRef wr = weight_ref(ly.down_weight, ly.down_scales, D, CI);
        fetch_rows<64, kIChunksPerLane>(wr, gw < D ? gw : D, lane, wreg + kSlotsLo * 64, sd);
    };

    if (cw >= 0) qkv_fetch(p.layers[0]);

    // ------------------------------------------------------------------- layers
    for (int l = 0; l < p.L; ++l) {
        const OrtmiDecoderLayer& ly = p.layers[l];
        // Phase A: input norm (+ residual), merged QKV GEMV.
        if (l == 0) {
            norm_stage<0>(p.embed + id * D, false, static_cast<const half_t*>(ly.ln1_gamma),
                          ly.ln1_epsilon, D, sR, sA, sRed);
        } else {
            norm_stage<kSC1>(p.dout, true, static_cast<const half_t*>(ly.ln1_gamma),
                             ly.ln1_epsilon, D, sR, sA, sRed);
        }
        if (cw >= 0) {
            const int ng = (NQ + 3) / 4;
            __builtin_amdgcn_s_waitcnt(0);
            float v = group_sum<16>(row_dot<16, CPLD>(wreg, sq, sA, CD, li16));
            if (gw < ng && li16 == 0 && 4 * gw + grp < NQ)
                st_half_sc1(p.qkv, (uint32_t)NQ * 2, 4 * gw + grp, v);
            __builtin_amdgcn_s_waitcnt(0);
            kv_fetch(ly);
            o_fetch(ly);
        }
        if (!grid_sync(bar, nwg, &s_flag, p.status)) return;
        if (bar.round == 1 && wg == 0 && tid == 0) {
            // Every workgroup read the parity before arriving here: reset the other
            // counter set for the next launch and flip the parity.
            const int other = bar.set ^ 1;
            store_dev(p.ctl + ctl_top(other), 0u);
            for (int x = 0; x < kXcds; ++x) store_dev(p.ctl + ctl_xcd(other, x), 0u);
            store_dev(p.ctl + kCtlParity, (unsigned)other);
        }

        // Phase B: attention (KV * NS workgroups), split partials. The query heads
        // of the KV group are taken HP at a time over the same K/V rows in LDS,
        // which bounds the per-lane softmax state.
        if (attn_wg) {
            constexpr int HP = G < 2 ? G : 2;
            const __amdgpu_buffer_rsrc_t rq = rsrc(p.qkv, (uint32_t)NQ * 2);
            const half_t* cs = p.half ? p.cos + (size_t)ctx * p.half : nullptr;
            const half_t* sn = p.half ? p.sin + (size_t)ctx * p.half : nullptr;
            if (cw >= 0) {
                __builtin_amdgcn_s_waitcnt(0);
                float kn[8], vn[8];
                uint32_t knw[4];
                const uint4 kraw = ld128<kSC1>(rq, (uint32_t)((H + a_kvh) * HD + li16 * 8) * 2u);
                const uint4 vraw =
                    ld128<kSC1>(rq, (uint32_t)((H + KV + a_kvh) * HD + li16 * 8) * 2u);
                const half_t* kh = reinterpret_cast<const half_t*>(&kraw);
                const half_t* vh = reinterpret_cast<const half_t*>(&vraw);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    kn[e] = (float)kh[e];
                    vn[e] = (float)vh[e];
                }
                rope8(kn, li16, p.half, cs, sn);
                half_t k8[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) k8[e] = (half_t)kn[e];
#pragma unroll
                for (int e = 0; e < 4; ++e) knw[e] = reinterpret_cast<const uint32_t*>(k8)[e];
                // The split holding the new key appends it to the cache (shared
                // buffer, written in place at row ctx).
                if (cw == 0 && grp == 0 && ctx >= k0 && ctx < k1) {
                    const size_t off = ((size_t)(a_kvh * p.cap + ctx) * HD + li16 * 8);
                    *reinterpret_cast<uint4*>(static_cast<half_t*>(ly.k_cache) + off) =
                        *reinterpret_cast<const uint4*>(k8);
                    *reinterpret_cast<uint4*>(static_cast<half_t*>(ly.v_cache) + off) = vraw;
                }
                const float qscale = p.scale * 1.4426950408889634f;  // scores in log2 units
                const int steps = (k1 - k0 + kKeySlots - 1) / kKeySlots;
                const uint32_t bytes = (uint32_t)KV * p.cap * HD * 2;
                const __amdgpu_buffer_rsrc_t rk = rsrc(ly.k_cache, bytes),
                                             rv = rsrc(ly.v_cache, bytes);
                for (int g0 = 0; g0 < G; g0 += HP) {
                    AttnState<HP> st;
                    uint32_t qh[HP][4];
#pragma unroll
                    for (int g = 0; g < HP; ++g) {
                        st.m[g] = -INFINITY;
                        st.l[g] = 0.f;
#pragma unroll
                        for (int e = 0; e < 8; ++e) st.o[g][e] = 0.f;
                        const int head = a_kvh * G + g0 + g;
                        const uint4 raw = ld128<kSC1>(rq, (uint32_t)(head * HD + li16 * 8) * 2u);
                        const half_t* rh = reinterpret_cast<const half_t*>(&raw);
                        float x[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[e] = (float)rh[e];
                        rope8(x, li16, p.half, cs, sn);
                        half_t q8[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) q8[e] = (half_t)x[e];
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            qh[g][e] = reinterpret_cast<const uint32_t*>(q8)[e];
                    }
                    auto attend = [&](const uint4& kr, const uint4& vr, int key) {
                        if (key >= k1) return;
                        const bool fresh = key == ctx;
                        const uint32_t kw[4] = {fresh ? knw[0] : kr.x, fresh ? knw[1] : kr.y,
                                                fresh ? knw[2] : kr.z, fresh ? knw[3] : kr.w};
                        float vv[8];
                        const half_t* vb = reinterpret_cast<const half_t*>(&vr);
#pragma unroll
                        for (int e = 0; e < 8; ++e) vv[e] = fresh ? vn[e] : (float)vb[e];
#pragma unroll
                        for (int g = 0; g < HP; ++g) {
                            float d = 0.f;
#pragma unroll
                            for (int e = 0; e < 4; ++e)
                                d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, qh[g][e]),
                                                           __builtin_bit_cast(half2_t, kw[e]), d,
                                                           false);
                            const float sc = group_sum<16>(d) * qscale;
                            const float mn = fmaxf(st.m[g], sc);
                            const float f = st.m[g] == -INFINITY ? 0.f : exp2f(st.m[g] - mn);
                            const float pe = exp2f(sc - mn);
                            st.l[g] = st.l[g] * f + pe;
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                st.o[g][e] = fmaf(pe, vv[e], st.o[g][e] * f);
                            st.m[g] = mn;
                        }
                    };
#pragma unroll
                    for (int t = 0; t < kPrefSteps; ++t)
                        if (t < steps)
                            attend(wreg[t * 64 + lane], wreg[(kPrefSteps + t) * 64 + lane],
                                   k0 + t * kKeySlots + slot);
                    for (int t = kPrefSteps; t < steps; ++t) {
                        const int key = k0 + t * kKeySlots + slot;
                        const bool ok = key < k1 && key < ctx;
                        const uint32_t off =
                            ok ? ((uint32_t)(a_kvh * p.cap + key) * HD + li16 * 8) * 2u : bytes;
                        attend(ld128<0>(rk, off), ld128<0>(rv, off), key);
                    }
                    // Merge the 4 lane groups of the wave (same dims, other keys).
#pragma unroll
                    for (int g = 0; g < HP; ++g) {
#pragma unroll
                        for (int sh = 16; sh <= 32; sh <<= 1) {
                            const float om = __shfl_xor(st.m[g], sh, 64);
                            const float ol = __shfl_xor(st.l[g], sh, 64);
                            const float mn = fmaxf(st.m[g], om);
                            const float fa = st.m[g] == -INFINITY ? 0.f : exp2f(st.m[g] - mn);
                            const float fb = om == -INFINITY ? 0.f : exp2f(om - mn);
                            st.l[g] = st.l[g] * fa + ol * fb;
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                const float oo = __shfl_xor(st.o[g][e], sh, 64);
                                st.o[g][e] = st.o[g][e] * fa + oo * fb;
                            }
                            st.m[g] = mn;
                        }
                        if (lane == 0) {
                            s_am[cw][g0 + g] = st.m[g];
                            s_al[cw][g0 + g] = st.l[g];
                        }
                        if (grp == 0) {
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                sO[(cw * kGMax + g0 + g) * HD + li16 * 8 + e] = st.o[g][e];
                        }
                    }
                }
            }
            __syncthreads();
            // Merge the 7 waves, write the split's partial per head: o[HD], m, l
            // (records of HD + 4 floats keep every record 16-byte aligned).
            const int stride = HD + 4;
            for (int idx = tid; idx < G * HD; idx += kThreads) {
                const int g = idx / HD, d = idx % HD;
                float M = -INFINITY;
#pragma unroll
                for (int w = 0; w < kComputeWaves; ++w) M = fmaxf(M, s_am[w][g]);
                float Lsum = 0.f, acc = 0.f;
#pragma unroll
                for (int w = 0; w < kComputeWaves; ++w) {
                    const float mw = s_am[w][g];
                    const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
                    Lsum += s_al[w][g] * f;
                    acc += sO[(w * kGMax + g) * HD + d] * f;
                }
                float* dst = p.part + ((size_t)(a_kvh * G + g) * kNSMax + a_split) * stride;
                __hip_atomic_store(dst + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (d == 0) {
                    __hip_atomic_store(dst + HD, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    __hip_atomic_store(dst + HD + 1, Lsum, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            __syncthreads();  // sO aliases sA, which the next phase restages
        }
        if (cw >= 0) {
            __builtin_amdgcn_s_waitcnt(0);
            gu_fetch(ly);
        }
        if (!grid_sync(bar, nwg, &s_flag, p.status)) return;

        // Phase C: merge the splits into the attention output (fp16), o_proj GEMV.
        {
            const int stride = HD + 4;
            const uint32_t pbytes = (uint32_t)H * kNSMax * stride * 4;
            const __amdgpu_buffer_rsrc_t rp = rsrc(p.part, pbytes);
            for (int t = tid; t < H * HD / 8; t += kThreads) {
                const int h = (t * 8) / HD, d0 = (t * 8) % HD;
                float ms[kNSMax], ls[kNSMax];
                float M = -INFINITY;
#pragma unroll
                for (int sidx = 0; sidx < kNSMax; ++sidx) {
                    const uint32_t rec = ((uint32_t)(h * kNSMax + sidx) * stride) * 4u;
                    const bool live = sidx < NS;
                    const uint4 ml = ld128<kSC1>(rp, live ? rec + (uint32_t)HD * 4u : pbytes);
                    ms[sidx] = live ? __uint_as_float(ml.x) : -INFINITY;
                    ls[sidx] = live ? __uint_as_float(ml.y) : 0.f;
                    M = fmaxf(M, ms[sidx]);
                }
                float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                float Lsum = 0.f;
#pragma unroll
                for (int sidx = 0; sidx < kNSMax; ++sidx) {
                    if (sidx >= NS) break;
                    const uint32_t rec = ((uint32_t)(h * kNSMax + sidx) * stride) * 4u;
                    const uint4 o0 = ld128<kSC1>(rp, rec + (uint32_t)d0 * 4u);
                    const uint4 o1 = ld128<kSC1>(rp, rec + (uint32_t)(d0 + 4) * 4u);
                    const float w = ms[sidx] == -INFINITY ? 0.f : exp2f(ms[sidx] - M);
                    Lsum += w * ls[sidx];
                    const float ov[8] = {__uint_as_float(o0.x), __uint_as_float(o0.y),
                                         __uint_as_float(o0.z), __uint_as_float(o0.w),
                                         __uint_as_float(o1.x), __uint_as_float(o1.y),
                                         __uint_as_float(o1.z), __uint_as_float(o1.w)};
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc[e] = fmaf(ov[e], w, acc[e]);
                }
                const float inv = Lsum > 0.f ? 1.0f / Lsum : 0.f;
                half_t o8[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) o8[e] = (half_t)(acc[e] * inv);
                sA[t] = permute_act8(*reinterpret_cast<const uint4*>(o8));
            }
            __syncthreads();
        }
        if (cw >= 0) {
            const int ng = (D + 3) / 4;
            __builtin_amdgcn_s_waitcnt(0);
            float v = group_sum<16>(row_dot<16, CPLD>(wreg + kSlotsLo * 64, so, sA, CO, li16));
            if (gw < ng && li16 == 0 && 4 * gw + grp < D)
                st_half_sc1(p.y, (uint32_t)D * 2, 4 * gw + grp, v);
            __builtin_amdgcn_s_waitcnt(0);
            down_fetch(ly);
        }
        if (!grid_sync(bar, nwg, &s_flag, p.status)) return;

        // Phase D: residual + post-attention norm, gate/up GEMV with SwiGLU.
        norm_stage<kSC1>(p.y, true, static_cast<const half_t*>(ly.ln2_gamma), ly.ln2_epsilon,
                         D, sR, sA, sRed);
        if (cw >= 0) {
            const int N = 2 * I, ng = (N + 3) / 4;
            auto gu_out = [&](float v, int g) {
                v = group_sum<16>(v);
                const float other = __shfl_xor(v, 16, 64);  // gate (even group) <-> up (odd)
                if (g < ng && li16 == 0 && (grp & 1) == 0) {
                    const int pair = 2 * g + (grp >> 1);
                    if (pair < I) {
                        const float gv = r16(v), up = r16(other);
                        const float sig = r16(1.0f / (1.0f + __expf(-gv)));
                        st_half_sc1(p.act, (uint32_t)I * 2, pair, r16(r16(gv * sig) * up));
                    }
                }
            };
            __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
            for (int k = 0; k < kGu; ++k)
                gu_out(row_dot<16, CPLD>(wreg + k * CPLD * 64, sg[k], sA, CD, li16), gw + k * TW);
            const WeightRef wr = weight_ref(ly.gate_up_weight, ly.gate_up_scales, N, CD);
            for (int g = gw + kGu * TW; g < ng; g += TW) {
                Rows<CPLD> r;
                load_rows<16, CPLD>(r, wr, 4 * g + grp, li16);
                gu_out(rows_dot<16, CPLD>(r, sA, CD, li16), g);
            }
            __builtin_amdgcn_s_waitcnt(0);
            if (l + 1 < p.L) qkv_fetch(p.layers[l + 1]);
        }
        if (!grid_sync(bar, nwg, &s_flag, p.status)) return;

        // Phase E: down GEMV (K = I).
        stage_vec(p.act, I, sA);
        if (cw >= 0) {
            __builtin_amdgcn_s_waitcnt(0);
            const float v = wave_sum(row_dot<64, kIChunksPerLane>(wreg + kSlotsLo * 64, sd, sA, CI, lane));
            if (gw < D && lane == 0) st_half_sc1(p.dout, (uint32_t)D * 2, gw, v);
        }
        if (!grid_sync(bar, nwg, &s_flag, p.status)) return;
    }

    // Phase F: final norm, lm_head GEMV (logits), per-workgroup argmax.
    norm_stage<kSC1>(p.dout, true, p.final_gamma, p.final_eps, D, sR, sA, sRed);
    float best = -INFINITY;
    int bi = -1;
    if (cw >= 0) {
        constexpr int kRing = 4;
        const int lm_ng = (p.V + 3) / 4;
        const WeightRef wr = weight_ref(p.lm_w, p.lm_s, p.V, CD);
        Rows<CPLD> ring[kRing];
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            const int g = gw + r * TW;
            load_rows<16, CPLD>(ring[r], wr, g < lm_ng ? 4 * g + grp : p.V, li16);
        }
        for (int k = 0;; k += kRing) {
            bool done = false;
#pragma unroll
            for (int r = 0; r < kRing; ++r) {
                const int g = gw + (k + r) * TW;
                if (g >= lm_ng) {
                    done = true;
                    break;
                }
                const float v = group_sum<16>(rows_dot<16, CPLD>(ring[r], sA, CD, li16));
                const int gn = g + kRing * TW;
                load_rows<16, CPLD>(ring[r], wr, gn < lm_ng ? 4 * gn + grp : p.V, li16);
                const int n = 4 * g + grp;
                if (n < p.V) {
                    const half_t hv = (half_t)v;
                    if (li16 == 0) p.logits[n] = hv;
                    const float fv = (float)hv;
                    if (fv > best || (bi < 0 && fv == best)) {
                        best = fv;
                        bi = n;
                    }
                }
            }
            if (done) break;
        }
    }
    // Reduce (value, index) over the workgroup: lowest index wins ties, NaN never wins.
    {
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) {
            const float ov = __shfl_xor(best, sh, 64);
            const int oi = __shfl_xor(bi, sh, 64);
            if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
                best = ov;
                bi = oi;
            }
        }
        if (lane == 0) {
            s_arg_v[wave] = best;
            s_arg_i[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 0; w < kThreads / 64; ++w) {
                const float ov = s_arg_v[w];
                const int oi = s_arg_i[w];
                if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
                    best = ov;
                    bi = oi;
                }
            }
            float4 rec = make_float4(best, __int_as_float(bi), 0.f, 0.f);
            st128<kSC1>(rsrc(p.argp, (uint32_t)nwg * 16), (uint32_t)wg * 16,
                        *reinterpret_cast<const uint4*>(&rec));
        }
    }
    if (!grid_sync(bar, nwg, &s_flag, p.status)) return;
    if (wg == 0) {
        best = -INFINITY;
        bi = -1;
        const __amdgpu_buffer_rsrc_t ra = rsrc(p.argp, (uint32_t)nwg * 16);
        for (int w = tid; w < nwg; w += kThreads) {
            const uint4 raw = ld128<kSC1>(ra, (uint32_t)w * 16);
            const float ov = __uint_as_float(raw.x);
            const int oi = (int)raw.y;
            if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
                best = ov;
                bi = oi;
            }
        }
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) {
            const float ov = __shfl_xor(best, sh, 64);
            const int oi = __shfl_xor(bi, sh, 64);
            if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
                best = ov;
                bi = oi;
            }
        }
        __syncthreads();
        if (lane == 0) {
            s_arg_v[wave] = best;
            s_arg_i[wave] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            for (int w = 0; w < kThreads / 64; ++w) {
                const float ov = s_arg_v[w];
                const int oi = s_arg_i[w];
                if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
                    best = ov;
                    bi = oi;
                }
            }
            *p.next_id = bi < 0 ? 0 : bi;
            store_status(p.status, bad_id ? 2 : 0);
        }
    }
}

}  // namespace dprog
}  // namespace ortmi

using namespace ortmi;

namespace {

struct StepShape {
    size_t ctl, qkv, part, y, act, dout, argp, total;
};

StepShape step_layout(const OrtmiDecoderDims* d, int nwg) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    StepShape s{};
    size_t off = 0;
    s.ctl = off;
    off += dprog::kCtlBytes;
    s.qkv = off;
    off += al((size_t)(d->num_heads + 2 * d->kv_num_heads) * d->head_size * 2);
    s.part = off;
    off += al((size_t)d->num_heads * dprog::kNSMax * (d->head_size + 4) * 4);
    s.y = off;
    off += al((size_t)d->hidden * 2);
    s.act = off;
    off += al((size_t)d->intermediate * 2);
    s.dout = off;
    off += al((size_t)d->hidden * 2);
    s.argp = off;
    off += al((size_t)nwg * 16);
    s.total = off;
    return s;
}

int program_grid() {
    const int cus = device_cu_count();
    return cus - cus % kXcds;
}

}  // namespace

extern "C" size_t ortmi_decoder_decode_step_workspace_size(const OrtmiDecoderDims* dims) {
    if (!dims) return 0;
    return step_layout(dims, program_grid()).total;
}

extern "C" int ortmi_decoder_decode_step(const OrtmiDecoderLayer* layers, const OrtmiDecoderDims* dims,
                                         const void* embed, int64_t embed_rows,
                                         const int64_t* input_id,
                                         const int32_t* total_sequence_length,
                                         const void* cos_cache, const void* sin_cache,
                                         const void* final_gamma, float final_epsilon,
                                         const uint8_t* lm_weight, const void* lm_scales,
                                         void* logits, int64_t* next_id, int32_t* status,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    ORTMI_REQUIRE(layers && dims && embed && input_id && total_sequence_length && final_gamma &&
                      lm_weight && lm_scales && logits && next_id && workspace,
                  "decoder step: null argument");
    const OrtmiDecoderDims& d = *dims;
    ORTMI_REQUIRE(d.dtype == ORTMI_F16, "decoder step: fp16 only");
    ORTMI_REQUIRE(d.block_size == 32, "decoder step: block size 32 only");
    ORTMI_REQUIRE(d.layers >= 1, "decoder step: no layers");
    ORTMI_REQUIRE(d.head_size == 128, "decoder step: head size 128 only");
    ORTMI_REQUIRE(d.num_heads > 0 && d.kv_num_heads > 0 && d.num_heads % d.kv_num_heads == 0 &&
                      d.num_heads / d.kv_num_heads <= dprog::kGMax,
                  "decoder step: at most 8 query heads per KV head");
    ORTMI_REQUIRE(d.hidden % 256 == 0 && d.hidden <= 2048, "decoder step: hidden % 256 == 0, <= 2048");
    ORTMI_REQUIRE((d.num_heads * d.head_size) % 256 == 0 && d.num_heads * d.head_size <= 2048,
                  "decoder step: num_heads * head_size % 256 == 0, <= 2048");
    ORTMI_REQUIRE(d.intermediate % 32 == 0 && d.intermediate <= 64 * 32 * dprog::kIChunksPerLane,
                  "decoder step: intermediate % 32 == 0, <= 10240");
    ORTMI_REQUIRE(d.vocab > 0 && embed_rows > 0 && d.kv_capacity > 0, "decoder step: bad sizes");
    ORTMI_REQUIRE(d.rotary_half == 0 || (d.rotary_half % 8 == 0 && 2 * d.rotary_half <= d.head_size &&
                                          cos_cache && sin_cache && d.max_position > 0),
                  "decoder step: rotary half must be a multiple of 8, at most head_size / 2");
    ORTMI_REQUIRE(d.rotary_interleaved == 0, "decoder step: interleaved rotary is not supported");
    const int nwg = program_grid();
    ORTMI_REQUIRE(nwg >= kXcds, "decoder step: too few compute units");
    const int nq = (d.num_heads + 2 * d.kv_num_heads) * d.head_size;
    ORTMI_REQUIRE((nq + 3) / 4 <= dprog::kComputeWaves * nwg && (d.hidden + 3) / 4 <= dprog::kComputeWaves * nwg &&
                      d.hidden <= dprog::kComputeWaves * nwg,
                  "decoder step: projection rows exceed one group per wave");
    ORTMI_REQUIRE(d.kv_num_heads * dprog::kNSMax <= nwg, "decoder step: too many KV heads");
    ORTMI_REQUIRE((int64_t)d.kv_num_heads * d.kv_capacity * d.head_size * 2 < (int64_t)INT32_MAX &&
                      (int64_t)d.vocab * d.hidden / 2 < (int64_t)INT32_MAX,
                  "decoder step: a cache or the lm_head exceeds 2 GiB");
    const StepShape s = step_layout(dims, nwg);
    if (workspace_bytes < s.total)
        return fail(ORTMI_E_WORKSPACE, "decoder step: workspace too small");
    ORTMI_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0 &&
                      (reinterpret_cast<uintptr_t>(embed) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(final_gamma) & 15) == 0,
                  "decoder step: workspace, embedding and gamma must be 16-byte aligned");

    char* ws = static_cast<char*>(workspace);
    dprog::Params p{};
    p.layers = layers;
    p.L = d.layers;
    p.D = d.hidden;
    p.H = d.num_heads;
    p.KV = d.kv_num_heads;
    p.I = d.intermediate;
    p.V = d.vocab;
    p.cap = d.kv_capacity;
    p.max_pos = d.max_position;
    p.half = d.rotary_half;
    p.nwg = nwg;
    p.scale = d.scale != 0.f ? d.scale : 1.0f / sqrtf((float)d.head_size);
    p.final_eps = final_epsilon;
    p.embed = static_cast<const half_t*>(embed);
    p.embed_rows = embed_rows;
    p.input_id = input_id;
    p.total = total_sequence_length;
    p.cos = static_cast<const half_t*>(cos_cache);
    p.sin = static_cast<const half_t*>(sin_cache);
    p.final_gamma = static_cast<const half_t*>(final_gamma);
    p.lm_w = lm_weight;
    p.lm_s = static_cast<const half_t*>(lm_scales);
    p.logits = static_cast<half_t*>(logits);
    p.next_id = next_id;
    p.status = status;
    p.ctl = reinterpret_cast<uint32_t*>(ws + s.ctl);
    p.qkv = reinterpret_cast<half_t*>(ws + s.qkv);
    p.part = reinterpret_cast<float*>(ws + s.part);
    p.y = reinterpret_cast<half_t*>(ws + s.y);
    p.act = reinterpret_cast<half_t*>(ws + s.act);
    p.dout = reinterpret_cast<half_t*>(ws + s.dout);
    p.argp = reinterpret_cast<float4*>(ws + s.argp);

    const int cpld = d.hidden <= 1536 && d.num_heads * d.head_size <= 1536 ? 3 : 4;
    const int G = d.num_heads / d.kv_num_heads;
    const void* fn = nullptr;
#define ORTMI_DP(C, GG)                                                                 \
    if (cpld == C && G == GG) fn = (const void*)dprog::decode_program_kernel<128, C, GG>;
    ORTMI_DP(3, 1) ORTMI_DP(3, 2) ORTMI_DP(3, 4) ORTMI_DP(3, 6) ORTMI_DP(3, 8)
    ORTMI_DP(4, 1) ORTMI_DP(4, 2) ORTMI_DP(4, 4) ORTMI_DP(4, 6) ORTMI_DP(4, 8)
#undef ORTMI_DP
    ORTMI_REQUIRE(fn, "decoder step: query heads per KV head must be 1, 2, 4, 6 or 8");
    const int a_units = std::max(d.hidden, d.intermediate) / 8;
    const int o_units = dprog::kComputeWaves * dprog::kGMax * d.head_size / 4;
    const size_t lds = ((size_t)dprog::kComputeWaves * dprog::region_slots(cpld) * 64 +
                        (size_t)std::max(a_units, o_units) + d.hidden / 8) * 16;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, dprog::kThreads, lds) != hipSuccess ||
        per_cu < 1) {
        (void)hipGetLastError();
        return fail(ORTMI_E_INVALID, "decoder step: the program does not fit one workgroup per CU");
    }
    void* args[] = {&p};
    const hipError_t e = hipLaunchCooperativeKernel(fn, dim3(nwg), dim3(dprog::kThreads), args,
                                                    (unsigned)lds, as_stream(stream));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(ORTMI_E_HIP, std::string("decoder step: cooperative launch: ") +
                                     hipGetErrorString(e));
    }
    return ORTMI_OK;
}
