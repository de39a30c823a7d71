// Int4 decoder decode step as one persistent kernel ("decode program") for gfx950.
//
// One launch runs a whole one-token step of a Llama-style int4
// decoder: embedding row -> per layer [(Skip)SimplifiedLayerNorm, merged QKV
// MatMulNBits, GroupQueryAttention over the shared KV cache with in-op RoPE,
// o_proj MatMulNBits, SkipSimplifiedLayerNorm, gate/up MatMulNBits with SwiGLU,
// down MatMulNBits] -> final SkipSimplifiedLayerNorm -> lm_head MatMulNBits ->
// greedy argmax. The reference reaches the same one-dispatch-per-token shape with
// a shapeless mlx_compile trace of the decode graph (rust/src/compiled.rs:1-28,
// 503-822).
//
// Why one kernel: at batch 1 every MatMulNBits of this decoder moves 1.3-16 MB,
// which the GPU streams in 1-3 us, while a dependent kernel boundary costs about
// 1.5 us and each small kernel spends another 1-2 us filling and draining. The
// weights of the next phase do not depend on the activations, so every wave
// issues the loads of its share of the next phase's weights (straight into LDS)
// before it waits for that phase's input: the HBM latency hides behind the wait.
//
// Dataflow, no grid barrier. Every phase output (qkv, attention output, o_proj
// output, SwiGLU activations, down output) is a vector of tagged words in a
// buffer of its own per layer: fp16 value in the low half, the launch tag in the
// high half, written with one device-coherent (sc1) 32-bit store. A consumer
// thread reads the units (8 words) it needs with sc1 loads and reads again only
// those whose tags are not yet this launch's, so a phase waits for exactly the
// data it uses, one memory round trip after the last producer's store, with no
// store acknowledgement, counter or flag in between. Words are single-copy
// atomic, so no ordering between stores is needed. The tag comes from a launch
// counter every workgroup bumps once at entry (launches on one workspace run in
// stream order, so a launch's workgroups all read the same count / nwg), and
// every buffer word is rewritten by every launch, so a stale word always carries
// the previous launch's tag.
//
// Grid: one 512-thread workgroup per CU (at most one fits per CU, so on an
// otherwise idle device a plain launch makes them all resident at once; a
// cooperative launch guarantees it), 8 waves, all computing. Attention runs on
// the last H * NS workgroups, one (query head, key split) each; the projections
// run on the others. Every wait is bounded: a wait that sees no new data for
// 100 ms of the 100 MHz realtime clock writes its launch index to the abort word
// and status 1, and every other waiting thread leaves when it sees its own
// launch index there. A workgroup that finds its launch index in the abort word
// at entry leaves at once (the host can abort a launch before it starts). No
// thread waits on anything its own workgroup produces later, so the waits form a
// chain along the layer order and always end.
//
// Rounding follows the unfused ops of the fp16 graph: residual sums and
// normalised activations, MatMulNBits outputs, the RoPE'd query/key and the
// attention output are rounded to fp16 where the graph stores them; sums and
// softmax state are fp32.
#include <map>
#include <mutex>
#include <tuple>

#include "common.h"

namespace ortmi {
namespace dprog {

// Per-phase timestamps for profiling, compiled in only with -DORTMI_DPROG_STAMPS
// (onnxruntime-mlx_amd/dprog_stamps.py builds that variant): thread 0 of each
// workgroup writes the 100 MHz realtime clock to slot k of its row, read back with
// ortmi_decoder_decode_step_stamps. Slots: 0 start; per layer l at 1 + 8 l:
// projection workgroups +0 A input ready, +1 A output stored, +2 C input ready,
// +3 C stored, +4 D input ready, +5 D stored, +6 E input ready, +7 E stored;
// attention workgroups +2 q/k/v ready, +4 keys attended, +5 merged in the
// workgroup, +6 partials in hand, +3 output stored; 1 + 8 L lm_head input ready,
// 2 + 8 L lm_head done; the last slot kernel entry, the one before it the greedy
// id written (workgroup 0).
constexpr int kStampSlots = 256;
#ifdef ORTMI_DPROG_STAMPS
__device__ unsigned long long g_stamps[1024 * kStampSlots];
#define DPROG_STAMP(k)                                                                \
    do {                                                                              \
        if (threadIdx.x == 0 && (k) < kStampSlots)                                    \
            g_stamps[blockIdx.x * kStampSlots + (k)] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#else
#define DPROG_STAMP(k) \
    do {               \
    } while (0)
#endif

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kSC1 = 16;               // buffer cache policy: device-coherent (sc1)
constexpr int kGMax = 8;               // query heads per KV head
constexpr int kKvRing = 4;             // attention steps in flight in registers
constexpr int kIChunksPerLane = 5;     // down_proj: K = I <= 5 * 64 * 32 = 10240
constexpr int kMaxLayers = 64;
constexpr int kMaxUnits = 3;           // tagged vectors up to 3 * 512 units of 8 values
constexpr int kNSMax = 8;              // key splits per attention head
constexpr int kPartWords = 130;        // a split's partial: o[128], running max, sum
constexpr unsigned long long kDeadlineTicks = 10000000ull;  // 100 ms

// Control block (uint32 words, one 128-byte line each).
constexpr int kCtlStart = 0;   // workgroups started, summed over launches (64-bit)
constexpr int kCtlAbort = 32;  // launch index + 1 of a launch that gave up
constexpr size_t kCtlBytes = 256;

struct Params {
    const OrtmiDecoderLayer* layers;
    int L, D, H, KV, G, I, V, cap, max_pos, half, nwg;
    int gq, go, ggu, gd;  // QKV / o_proj / gate-up groups and down rows per workgroup
    int nc, ns;           // projection workgroups; key splits per attention head
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
    uint32_t* flow;          // per layer: qkv [NQ], att [H*hd], y [D], act [I], dout [D]
    uint32_t flow_stride;    // words per layer
    uint64_t* part;          // per layer: attention split partials [H][NS][kPartWords]
    uint64_t* argp;          // per workgroup: index | fp16 value << 32 | tag << 48
};

// A pointer every lane of the wave holds, made provably uniform (scalar registers):
// pointers read from the layer table in LDS arrive in vector registers, and a
// buffer resource built from those would make every load a per-lane loop.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(uniform_ptr(p)), 0,
                                             (int)__builtin_amdgcn_readfirstlane(bytes), kBufferWord3);
}
template <int POL>
__device__ __forceinline__ uint2 ld64(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, POL));
}
template <int POL>
__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POL);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ unsigned long long atomic_add_dev64(unsigned long long* p,
                                                               unsigned long long v) {
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
// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt at their maxima).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// ------------------------------------------------------------ tagged data
struct Flow {
    uint32_t* ctl;
    int32_t* status;
    uint32_t tag;     // 1..65535, in the high half of every data word
    uint32_t launch;  // launch index + 1 (32 bits), what the abort word holds
};

// One round of a bounded wait: false when this launch stops (another workgroup
// gave up, or this wait saw no data for 100 ms and gives up). `t0` is the wait's
// start on the realtime clock, taken at its first round, so the bound is per wait
// and a long step that keeps making progress is never cut short.
__device__ __forceinline__ bool keep_waiting(const Flow& f, unsigned it, unsigned long long& t0) {
    const unsigned long long now = __builtin_amdgcn_s_memrealtime();
    if (it == 0) t0 = now;
    if ((it & 7) == 7 && load_dev(f.ctl + kCtlAbort) == f.launch) return false;
    if (now - t0 > kDeadlineTicks) {
        store_dev(f.ctl + kCtlAbort, f.launch);
        store_status(f.status, 1);
        return false;
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

__device__ __forceinline__ bool tags_ok(const uint4& a, const uint4& b, uint32_t tag) {
    return ((a.x >> 16) == tag) & ((a.y >> 16) == tag) & ((a.z >> 16) == tag) &
           ((a.w >> 16) == tag) & ((b.x >> 16) == tag) & ((b.y >> 16) == tag) &
           ((b.z >> 16) == tag) & ((b.w >> 16) == tag);
}
// The fp16 halves of 8 tagged words, in order.
__device__ __forceinline__ uint4 untag(const uint4& a, const uint4& b) {
    return make_uint4(__builtin_amdgcn_perm(a.y, a.x, 0x05040100u),
                      __builtin_amdgcn_perm(a.w, a.z, 0x05040100u),
                      __builtin_amdgcn_perm(b.y, b.x, 0x05040100u),
                      __builtin_amdgcn_perm(b.w, b.z, 0x05040100u));
}

// Waits until the 8-word units at byte offsets off[k] (those with bit k of
// `pend`) carry this launch's tag and returns their fp16 values. Offsets of units
// not wanted lie past the buffer (they read zeros and touch no memory). False:
// the launch stops.
template <int N>
__device__ __forceinline__ bool poll_units(__amdgpu_buffer_rsrc_t r, const uint32_t (&off)[N],
                                           unsigned pend, const Flow& f, uint4 (&out)[N]) {
    uint4 lo[N], hi[N];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        lo[k] = ld128<kSC1>(r, off[k]);
        hi[k] = ld128<kSC1>(r, off[k] + 16u);
    }
    unsigned long long t0 = 0;
    for (unsigned it = 0;; ++it) {
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (((pend >> k) & 1u) && tags_ok(lo[k], hi[k], f.tag)) {
                out[k] = untag(lo[k], hi[k]);
                pend &= ~(1u << k);
            }
        if (!pend) return true;
        if (!keep_waiting(f, it, t0)) return false;
#pragma unroll
        for (int k = 0; k < N; ++k)
            if ((pend >> k) & 1u) {
                lo[k] = ld128<kSC1>(r, off[k]);
                hi[k] = ld128<kSC1>(r, off[k] + 16u);
            }
    }
}

// Tagged store of one fp16 value.
__device__ __forceinline__ void put(__amdgpu_buffer_rsrc_t r, int idx, float v, uint32_t tag) {
    __builtin_amdgcn_raw_buffer_store_b32(f2h(v) | (tag << 16), r, (uint32_t)idx * 4u, 0, kSC1);
}

// Every thread of the workgroup calls this after its own waits: true when no
// thread of the workgroup gave up.
__device__ __forceinline__ bool all_ok(bool ok, int* s_fail) {
    if (!ok) *s_fail = 1;
    __syncthreads();
    return *s_fail == 0;
}

// Sum of the 8 fp16 values of a unit, and (on the first lane of each 4 lanes) the
// sum over the 32-value chunk those 4 consecutive lanes hold, into sSum[chunk].
__device__ __forceinline__ void chunk_sum(uint4 v, bool valid, int unit, float* sSum) {
    const half_t* h = reinterpret_cast<const half_t*>(&v);
    float t = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) t += (float)h[e];
    t = group_sum<4>(valid ? t : 0.f);
    if (valid && (unit & 3) == 0) sSum[unit >> 2] = t;
}

// Stage a tagged fp16 vector of n values (n % 32 == 0, n <= kMaxUnits * 4096) into
// LDS in pair order, with its 32-value chunk sums in sSum. The caller has passed a
// workgroup barrier since sA and sSum were last read.
__device__ __forceinline__ bool stage_poll(const uint32_t* src, int n, uint4* sA, float* sSum,
                                           const Flow& f, int* s_fail) {
    const int units = n / 8;
    const uint32_t bytes = (uint32_t)n * 4u;
    uint32_t off[kMaxUnits];
    unsigned pend = 0;
#pragma unroll
    for (int k = 0; k < kMaxUnits; ++k) {
        const int u = threadIdx.x + k * kThreads;
        off[k] = u < units ? (uint32_t)u * 32u : bytes;
        if (u < units) pend |= 1u << k;
    }
    uint4 v[kMaxUnits];
    const bool ok = poll_units<kMaxUnits>(rsrc(src, bytes), off, pend, f, v);
#pragma unroll
    for (int k = 0; k < kMaxUnits; ++k) {
        const int u = threadIdx.x + k * kThreads;
        if (ok && u < units) sA[u] = permute_act8(v[k]);
        chunk_sum(v[k], ok && u < units, u, sSum);
    }
    return all_ok(ok, s_fail);
}

// Residual add + RMS norm of one D-vector (D <= 4096) into LDS: r = fp16(in +
// r_prev) (r = in when r_prev is not added), a = fp16(r * rsqrt(mean(r^2) + eps)
// * gamma); r kept in sR, a staged in pair order in sA. `in` is a tagged vector
// (src) or a constant fp16 row.
__device__ __forceinline__ bool norm_poll(const uint32_t* src, const half_t* row, bool add_prev,
                                          const half_t* gamma, float eps, int D, uint4* sR,
                                          uint4* sA, float* sSum, float* sRed, const Flow& f,
                                          int* s_fail) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int units = D / 8;
    const bool mine = tid < units;
    // A buffer load (the pointer comes from LDS, so a plain load would be a flat one,
    // which also counts against the LDS counter).
    const uint4 gv = ld128<0>(rsrc(gamma, (uint32_t)D * 2u), mine ? (uint32_t)tid * 16u : (uint32_t)D * 2u);
    uint4 v = make_uint4(0, 0, 0, 0);
    bool ok = true;
    if (src) {
        const uint32_t bytes = (uint32_t)D * 4u;
        const uint32_t off[1] = {mine ? (uint32_t)tid * 32u : bytes};
        uint4 out[1];
        ok = poll_units<1>(rsrc(src, bytes), off, mine ? 1u : 0u, f, out);
        v = out[0];
    } else if (mine) {
        v = reinterpret_cast<const uint4*>(row)[tid];
    }
    float ss = 0.f;
    if (mine && ok) {
        if (add_prev) {
            const uint4 pv = sR[tid];
            const half_t* a = reinterpret_cast<const half_t*>(&v);
            const half_t* b = reinterpret_cast<const half_t*>(&pv);
            half_t t[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) t[e] = (half_t)((float)a[e] + (float)b[e]);
            v = *reinterpret_cast<const uint4*>(t);
        }
        sR[tid] = v;
        const half_t* t = reinterpret_cast<const half_t*>(&v);
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += (float)t[e] * (float)t[e];
    }
    ss = wave_sum(ss);
    if (lane == 0) sRed[wave] = ss;
    if (!all_ok(ok, s_fail)) return false;
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tot += sRed[w];
    const float scale = 1.0f / sqrtf(tot / (float)D + eps);
    uint4 ov = make_uint4(0, 0, 0, 0);
    if (mine) {
        const half_t* t = reinterpret_cast<const half_t*>(&v);
        const half_t* g = reinterpret_cast<const half_t*>(&gv);
        half_t o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (half_t)((float)t[e] * scale * (float)g[e]);
        ov = *reinterpret_cast<const uint4*>(o);
        sA[tid] = permute_act8(ov);
    }
    chunk_sum(ov, mine, tid, sSum);
    __syncthreads();
    return true;
}

// LPR lanes (dims 8*li .. 8*li+7 of one head of LPR * 8 dims) rotate their 8
// values, non-interleaved pairs (i, i + half) over dims [0, 2*half), with the
// cos/sin row cs/sn [half]; the partner lane is li +- half / 8 inside the same
// LPR-lane group (half is a multiple of 8 and at most 4 * LPR).
template <int LPR>
__device__ __forceinline__ void rope8(float (&x)[8], int li, int half, const float* cs,
                                      const float* sn) {
    if (half == 0) return;
    const int off = half / 8;
    float px[8];
    if (LPR == 16 && off == 8) {
        // Partner li ^ 8 inside the 16-lane row: a DPP row rotation by 8.
#pragma unroll
        for (int i = 0; i < 8; ++i) px[i] = dpp_mov<0x128>(x[i]);
    } else {
        const int lane = threadIdx.x & 63;
        const int partner = (lane & ~(LPR - 1)) |
                            (((li < off || (li >= 2 * off)) ? li + off : li - off) & (LPR - 1));
#pragma unroll
        for (int i = 0; i < 8; ++i) px[i] = __shfl(x[i], partner & 63, 64);
    }
    const int d0 = li * 8;
    if (d0 >= 2 * half) return;
    const bool low = d0 < half;
    const int b = low ? d0 : d0 - half;
#pragma unroll
    for (int i = 0; i < 8; ++i)
        x[i] = low ? x[i] * cs[b + i] - px[i] * sn[b + i] : x[i] * cs[b + i] + px[i] * sn[b + i];
}

// An opaque copy of a per-lane value: what is computed from it inside a loop is
// recomputed there instead of being hoisted and held (or spilled) across the loop.
__device__ __forceinline__ int opaque(int v) {
    asm volatile("" : "+v"(v));
    return v;
}

// ------------------------------------------------------------ weight rows
// Row chunks of one phase are fetched straight into LDS (buffer_load_dwordx4
// ... lds: lane i's 16 bytes land at the slot base + 16 * i), so the weights a
// wave prefetches across a wait hold no registers. A wave owns kRegion slots of
// 64 x 16 bytes; the per-chunk fp16 scales stay in VGPRs. Chunk c = li + j * LPR
// of row n goes to slot `slot0 + j`; rows past N and chunks past C read zeros
// (offsets past the buffer ranges), so the loads are unconditional.
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

// sum(a * q) over one 32-code chunk. The codes are never converted: a 16-bit half
// whose bits are 0000 0000 qqqq 0000 or 0000 0000 0000 qqqq is the fp16 subnormal
// q * 2^-20 or q * 2^-24, so one AND per pair of codes, (w & 0x000F000F) for
// nibbles (j, j+4) and (w & 0x00F000F0) for (j+1, j+5), gives both operands of
// v_dot2_f32_f16 exactly (products exact, fp32 accumulation), and two exact
// power-of-two multiplies undo the scaling. The activations are in pair order
// (a_j, a_j+4), as permute_act8 stages them.
__device__ __forceinline__ float dot32_codes(const uint4 (&av)[4], uint4 w) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t aw[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
        const uint32_t x = words[i], y = words[i] >> 8;
        const uint32_t q[4] = {x & 0x000F000Fu, x & 0x00F000F0u, y & 0x000F000Fu, y & 0x00F000F0u};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const half2_t a = __builtin_bit_cast(half2_t, aw[j]);
            const half2_t b = __builtin_bit_cast(half2_t, q[j]);
            if (j & 1) d1 = __builtin_amdgcn_fdot2(a, b, d1, false);
            else d0 = __builtin_amdgcn_fdot2(a, b, d0, false);
        }
    }
    return d0 * 16777216.0f + d1 * 1048576.0f;
}

// Dot product of a lane's chunks (in LDS slots) with the staged activations (pair
// order, 4 uint4 per 32-code chunk; sSum the chunk sums), symmetric int4 (zero
// point 8): sum_j s_j * (sum(a * q) - 8 * sum(a)).
template <int LPR, int CPL>
__device__ __forceinline__ float row_dot(const uint4* slot0, const uint32_t (&sc)[CPL],
                                         const uint4* sA, const float* sSum, int C, int li) {
    const int lane = threadIdx.x & 63;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        if (c < C) {
            const uint4 av[4] = {sA[4 * c], sA[4 * c + 1], sA[4 * c + 2], sA[4 * c + 3]};
            acc = fmaf(h2f(sc[j]), fmaf(-8.f, sSum[c], dot32_codes(av, slot0[j * 64 + lane])), acc);
        }
    }
    return acc;
}

// NG row groups in LDS slots (group k's chunks at slot0 + k * CPL * 64) and NR
// register groups at once, into acc[0, NG) and acc[NG, NG + NR): each activation
// chunk is read from LDS once for all of them (read once per group, the three
// gate/up groups of the benchmark decoder took 2.80 us of D; at once 2.40 us). Per
// row the same products in the same order as row_dot / rows_dot.
template <int CPL>
struct Rows;
template <int LPR, int CPL, int NG, int NR>
__device__ __forceinline__ void rows_dot_multi(const uint4* slot0, const uint32_t (&sc)[NG][CPL],
                                               const Rows<CPL>* const (&rg)[NR > 0 ? NR : 1],
                                               const uint4* sA, const float* sSum, int C, int li,
                                               float (&acc)[NG + NR]);

// Register form for the lm_head stream and the gate/up groups beyond the
// prefetched ones: the chunks themselves in VGPRs.
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
__device__ __forceinline__ float rows_dot(const Rows<CPL>& r, const uint4* sA, const float* sSum,
                                          int C, int li) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        if (c < C) {
            const uint4 av[4] = {sA[4 * c], sA[4 * c + 1], sA[4 * c + 2], sA[4 * c + 3]};
            acc = fmaf(h2f(r.s[j]), fmaf(-8.f, sSum[c], dot32_codes(av, r.w[j])), acc);
        }
    }
    return acc;
}

template <int LPR, int CPL, int NG, int NR>
__device__ __forceinline__ void rows_dot_multi(const uint4* slot0, const uint32_t (&sc)[NG][CPL],
                                               const Rows<CPL>* const (&rg)[NR > 0 ? NR : 1],
                                               const uint4* sA, const float* sSum, int C, int li,
                                               float (&acc)[NG + NR]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < NG + NR; ++k) acc[k] = 0.f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = li + j * LPR;
        if (c < C) {
            const uint4 av[4] = {sA[4 * c], sA[4 * c + 1], sA[4 * c + 2], sA[4 * c + 3]};
            const float sm = sSum[c];
#pragma unroll
            for (int k = 0; k < NG; ++k)
                acc[k] = fmaf(h2f(sc[k][j]), fmaf(-8.f, sm, dot32_codes(av, slot0[(k * CPL + j) * 64 + lane])),
                              acc[k]);
#pragma unroll
            for (int k = 0; k < NR; ++k)
                acc[NG + k] = fmaf(h2f(rg[k]->s[j]), fmaf(-8.f, sm, dot32_codes(av, rg[k]->w[j])),
                                   acc[NG + k]);
        }
    }
}

// (value, index) argmax step: lowest index wins ties, a record without an index
// never wins, NaN never wins (comparisons with it are false).
__device__ __forceinline__ void arg_take(float& best, int& bi, float ov, int oi) {
    if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
        best = ov;
        bi = oi;
    }
}
__device__ __forceinline__ void arg_wave(float& best, int& bi) {
#pragma unroll
    for (int sh = 32; sh >= 1; sh >>= 1) arg_take(best, bi, __shfl_xor(best, sh, 64), __shfl_xor(bi, sh, 64));
}

constexpr int gu_groups(int cpld) { return cpld == 3 ? 3 : cpld == 4 ? 2 : 1; }
// Slot plan of a wave's LDS region (chunks of 64 x 16 bytes), projection
// workgroups, with the phase whose end requests each range:
//   gate/up [0, kGu * CPLD)        end of A      read in D
//   down [kLo, kLo + 5)            end of C      read in E
//   QKV [0, CPLD)                  end of D      read in A of the next layer
//   o_proj [kLo, kLo + CPLD)       end of E      read in C of the next layer
// Every range is written only after the wave consumed what it overlaps. Attention
// workgroups hold K [0, P) and V [P, 2P) of their key split, requested at the end
// of the previous layer's attention.
constexpr int region_lo(int cpld) { return gu_groups(cpld) * cpld; }
constexpr int region_slots(int cpld) {
    return region_lo(cpld) + (cpld > kIChunksPerLane ? cpld : kIChunksPerLane);
}
constexpr int kv_pref_steps(int cpld) { return region_slots(cpld) / 2; }

template <int HD, int CPLD>
__global__ __launch_bounds__(kThreads, 1) void decode_program_kernel(Params p) {
    extern __shared__ uint4 smem[];
    __shared__ OrtmiDecoderLayer s_layers[kMaxLayers];
    __shared__ float sRed[kWaves];
    __shared__ int s_fail;
    __shared__ uint32_t s_tag, s_launch;
    __shared__ int s_aborted;
    __shared__ float s_am[kWaves], s_al[kWaves];
    __shared__ float s_arg_v[kWaves];
    __shared__ int s_arg_i[kWaves];
    __shared__ float s_cos[64], s_sin[64];
    __shared__ float s_out[64];  // a phase's outputs of this workgroup, stored as one block
    __shared__ float s_pm[kNSMax], s_pl[kNSMax];  // sibling splits' running max and sum
    constexpr int kGu = gu_groups(CPLD);
    constexpr int kLo = region_lo(CPLD);
    constexpr int kRegion = region_slots(CPLD);
    constexpr int kPref = kv_pref_steps(CPLD);
    static_assert(kLo + CPLD <= kRegion && 2 * kPref <= kRegion, "slots");

    DPROG_STAMP(kStampSlots - 1);  // kernel entry
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
    const int wg = blockIdx.x, nwg = p.nwg;
    const int TW = kWaves * nwg;
    const int gw = wave * nwg + wg;  // global wave index (spreads the lm_head over CUs)
    const int D = p.D, H = p.H, KV = p.KV, I = p.I;
    const int NQ = (H + 2 * KV) * HD, HO = H * HD;
    const int CD = D / 32, CO = HO / 32, CI = I / 32;
    const int li16 = lane & 15, grp = lane >> 4;
    const int NC = p.nc;  // workgroups [0, NC) run the projections, [NC, nwg) attention
    const bool attn_wg = wg >= NC;

    // LDS: weight (or K/V) regions, activations (norm outputs; staged vectors),
    // residual, attention merge.
    uint4* wreg = smem + (size_t)wave * kRegion * 64;
    uint4* sA0 = smem + (size_t)kWaves * kRegion * 64;
    uint4* sA1 = sA0 + D / 8;
    uint4* sR = sA1 + (HO > I ? HO : I) / 8;
    float* sO = reinterpret_cast<float*>(sR + D / 8);  // [kWaves][HD]
    float* sSum0 = sO + kWaves * HD;                     // chunk sums of sA0 [D / 32]
    float* sSum1 = sSum0 + D / 32;                       // chunk sums of sA1

    if (tid == 0) s_fail = 0;
    {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(p.layers);
        uint32_t* dst = reinterpret_cast<uint32_t*>(s_layers);
        const int words = p.L * (int)(sizeof(OrtmiDecoderLayer) / 4);
        for (int i = tid; i < words; i += kThreads) dst[i] = src[i];
    }
    const int total = *p.total;
    if (total < 1 || total > p.cap || (p.half > 0 && total > p.max_pos)) {
        if (wg == 0 && tid == 0) store_status(p.status, 3);
        return;
    }
    if (tid == 0) {
        // A 64-bit count: the launch index stays the same for every workgroup of a
        // launch (a 32-bit count would wrap inside a launch unless nwg divides 2^32).
        const unsigned long long started =
            atomic_add_dev64(reinterpret_cast<unsigned long long*>(p.ctl + kCtlStart), 1ull);
        const unsigned long long li = started / (unsigned long long)nwg;
        s_tag = (uint32_t)(li % 65535ull) + 1u;
        s_launch = (uint32_t)li + 1u;
        s_aborted = load_dev(p.ctl + kCtlAbort) == s_launch;
    }
    const int ctx = total - 1;  // cached keys; the new key sits at index ctx
    if (attn_wg && tid < p.half) {
        s_cos[tid] = (float)p.cos[(size_t)ctx * p.half + tid];
        s_sin[tid] = (float)p.sin[(size_t)ctx * p.half + tid];
    }
    __syncthreads();
    if (s_aborted) return;  // aborted before it started: nothing is read or written
    const Flow f{p.ctl, p.status, s_tag, s_launch};
    const uint32_t tag = f.tag;
    DPROG_STAMP(0);

    int64_t id = *p.input_id;  // negative ids count from the end
    if (id < 0) id += p.embed_rows;
    const bool bad_id = id < 0 || id >= p.embed_rows;
    if (bad_id) id = 0;
    uint32_t* const f_res = p.flow + (size_t)p.L * p.flow_stride;  // last post-attention residual
    const uint32_t* prev_dout = p.flow + (size_t)(p.L - 1) * p.flow_stride + NQ + HO + 2 * D + I - D;

    if (attn_wg) {
        // ---------------------------------------------------- attention workgroups
        // Workgroup a = wg - NC owns keys [k0, k1) of query head h = a / NS. Its K/V
        // rows sit in LDS, requested right after the previous layer's attention, so
        // the wait for q/k/v never queues behind them. Split 0 of each head merges
        // the others' partials (tagged 64-bit words: value, tag) into the output.
        // A key row is LPR lanes of 8 dims (16 lanes for head 128, 8 for head 64;
        // head 96 takes 16-lane rows whose last 4 lanes hold no dims: their loads
        // read zeros and they store nothing); a wave holds GPW keys per step.
        constexpr int LPR = HD <= 64 ? 8 : 16, GPW = 64 / LPR, KEYS = kWaves * GPW;
        const int lr = lane % LPR, ag = lane / LPR;
        const bool padl = lr * 8 >= HD;
        const int NS = p.ns, a = wg - NC;
        const int h = a / NS, s = a % NS, kvh = h / p.G;
        const int ks = (total + NS - 1) / NS;
        const int k0 = s * ks, k1 = min(k0 + ks, total);
        const int steps = k1 > k0 ? (k1 - k0 + KEYS - 1) / KEYS : 0;
        const uint32_t kv_bytes = (uint32_t)KV * p.cap * HD * 2;
        const int slot = wave * GPW + ag;  // key slot of this lane group
        auto kv_off = [&](int t) -> uint32_t {
            const int key = k0 + slot + t * KEYS;
            return key < k1 && key < ctx && !padl
                       ? ((uint32_t)(kvh * p.cap + key) * HD + lr * 8) * 2u
                       : kv_bytes;
        };
        auto kv_fetch = [&](const OrtmiDecoderLayer& ly) {
            const __amdgpu_buffer_rsrc_t rk = rsrc(ly.k_cache, kv_bytes), rv = rsrc(ly.v_cache, kv_bytes);
#pragma unroll
            for (int t = 0; t < kPref; ++t) {
                const uint32_t off = kv_off(t);
                dma16(rk, off, wreg + t * 64);
                dma16(rv, off, wreg + (kPref + t) * 64);
            }
        };
        const float qscale = p.scale * 1.4426950408889634f;  // scores in log2 units
        kv_fetch(s_layers[0]);
        for (int l = 0; l < p.L; ++l) {
            const OrtmiDecoderLayer& ly = s_layers[l];
            uint32_t* f_qkv = p.flow + (size_t)l * p.flow_stride;
            uint32_t* f_att = f_qkv + NQ;
            uint64_t* f_part = p.part + (size_t)l * H * NS * kPartWords;
            const __amdgpu_buffer_rsrc_t rk = rsrc(ly.k_cache, kv_bytes), rv = rsrc(ly.v_cache, kv_bytes);
            // Steps past the LDS-resident ones (long contexts) go through a register ring.
            uint4 ringk[kKvRing], ringv[kKvRing];
            if (steps > kPref) {
#pragma unroll
                for (int r = 0; r < kKvRing; ++r) {
                    const uint32_t off = kv_off(kPref + r);
                    ringk[r] = ld128<kCachePolicyNT>(rk, off);
                    ringv[r] = ld128<kCachePolicyNT>(rv, off);
                }
            }
            const uint32_t off[3] = {(uint32_t)(h * HD + lr * 8) * 4u,
                                     (uint32_t)((H + kvh) * HD + lr * 8) * 4u,
                                     (uint32_t)((H + KV + kvh) * HD + lr * 8) * 4u};
            uint4 qkv3[3] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
            const uint32_t none = (uint32_t)NQ * 4u;
            const uint32_t offp[3] = {padl ? none : off[0], padl ? none : off[1], padl ? none : off[2]};
            const bool ok = poll_units<3>(rsrc(f_qkv, (uint32_t)NQ * 4u), offp, padl ? 0u : 7u, f, qkv3);
            DPROG_STAMP(1 + l * 8 + 2);
            float q[8], kn[8], vn[8];
            {
                const half_t* qh = reinterpret_cast<const half_t*>(&qkv3[0]);
                const half_t* kh = reinterpret_cast<const half_t*>(&qkv3[1]);
                const half_t* vh = reinterpret_cast<const half_t*>(&qkv3[2]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    q[e] = (float)qh[e];
                    kn[e] = (float)kh[e];
                    vn[e] = (float)vh[e];
                }
            }
            rope8<LPR>(q, lr, p.half, s_cos, s_sin);
            rope8<LPR>(kn, lr, p.half, s_cos, s_sin);
            uint32_t qw[4], kw_new[4];
            {
                half_t q8[8], k8[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    q8[e] = (half_t)q[e];
                    k8[e] = (half_t)kn[e];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    qw[e] = reinterpret_cast<const uint32_t*>(q8)[e];
                    kw_new[e] = reinterpret_cast<const uint32_t*>(k8)[e];
                }
            }
            // The split holding key ctx of the first query head of the KV group
            // appends the new key/value row to the cache (written in place at ctx).
            // Buffer stores (an offset past the caches when this lane does not append):
            // a flat store would also count against the LDS counter, and the LDS
            // reads below would wait for it to complete.
            {
                const bool app =
                    ok && h % p.G == 0 && ctx >= k0 && ctx < k1 && wave == 0 && ag == 0 && !padl;
                const uint32_t ao =
                    app ? (uint32_t)(((size_t)(kvh * p.cap + ctx) * HD + lr * 8) * 2) : kv_bytes;
                __builtin_amdgcn_raw_buffer_store_b128(
                    u32x4_t{kw_new[0], kw_new[1], kw_new[2], kw_new[3]}, rk, ao, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(
                    u32x4_t{qkv3[2].x, qkv3[2].y, qkv3[2].z, qkv3[2].w}, rv, ao, 0, 0);
            }
            float m = -INFINITY, lsum = 0.f, o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = 0.f;
            auto attend = [&](const uint4& kr, const uint4& vr, int key) {
                if (key >= k1) return;  // a whole LPR-lane group shares the key
                const bool fresh = key == ctx;
                const uint32_t kw[4] = {fresh ? kw_new[0] : kr.x, fresh ? kw_new[1] : kr.y,
                                        fresh ? kw_new[2] : kr.z, fresh ? kw_new[3] : kr.w};
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, qw[e]),
                                               __builtin_bit_cast(half2_t, kw[e]), d, false);
                const float sc = group_sum<LPR>(d) * qscale;
                const float mn = fmaxf(m, sc);
                const float fo = m == -INFINITY ? 0.f : exp2f(m - mn);
                const float pe = exp2f(sc - mn);
                lsum = lsum * fo + pe;
                const half_t* vb = reinterpret_cast<const half_t*>(&vr);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] = fmaf(pe, fresh ? vn[e] : (float)vb[e], o[e] * fo);
                m = mn;
            };
            // The LDS K/V rows were requested before the q/k/v words, and a wave's
            // vector memory requests complete in order: reading them through an
            // index that depends on the polled words orders the reads after both
            // (without also waiting for the cache-append stores above).
            int kv_lane = lane;
            asm volatile("" : "+v"(kv_lane) : "v"(qkv3[0].x), "v"(qkv3[2].w));
            // The LDS-resident keys as one block: every score first (independent
            // dot products and reductions), then one maximum and the weighted sum,
            // instead of a rescale chain through the keys one at a time.
            {
                float sc[kPref];
                float bmax = -INFINITY;
#pragma unroll
                for (int t = 0; t < kPref; ++t) {
                    sc[t] = -INFINITY;
                    if (t < steps) {
                        const int key = k0 + slot + t * KEYS;
                        const uint4 kr = wreg[t * 64 + kv_lane];
                        const bool fresh = key == ctx;
                        const uint32_t kw[4] = {fresh ? kw_new[0] : kr.x, fresh ? kw_new[1] : kr.y,
                                                fresh ? kw_new[2] : kr.z, fresh ? kw_new[3] : kr.w};
                        float d = 0.f;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            d = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, qw[e]),
                                                       __builtin_bit_cast(half2_t, kw[e]), d, false);
                        const float sv = group_sum<LPR>(d) * qscale;
                        sc[t] = key < k1 ? sv : -INFINITY;
                        bmax = fmaxf(bmax, sc[t]);
                    }
                }
                if (bmax != -INFINITY) {  // m is still -inf: no rescale
#pragma unroll
                    for (int t = 0; t < kPref; ++t) {
                        if (t < steps) {
                            const int key = k0 + slot + t * KEYS;
                            const float pe = sc[t] == -INFINITY ? 0.f : exp2f(sc[t] - bmax);
                            lsum += pe;
                            const uint4 vr = wreg[(kPref + t) * 64 + kv_lane];
                            const half_t* vb = reinterpret_cast<const half_t*>(&vr);
                            const bool fresh = key == ctx;
#pragma unroll
                            for (int e = 0; e < 8; ++e) o[e] = fmaf(pe, fresh ? vn[e] : (float)vb[e], o[e]);
                        }
                    }
                    m = bmax;
                }
            }
            for (int t0 = kPref; t0 < steps; t0 += kKvRing) {
#pragma unroll
                for (int r = 0; r < kKvRing; ++r) {
                    const int t = t0 + r;
                    if (t < steps) attend(ringk[r], ringv[r], k0 + slot + t * KEYS);
                    const uint32_t off2 = kv_off(t + kKvRing);
                    ringk[r] = ld128<kCachePolicyNT>(rk, off2);
                    ringv[r] = ld128<kCachePolicyNT>(rv, off2);
                }
            }
            DPROG_STAMP(1 + l * 8 + 4);
            // Merge the GPW lane groups of the wave (same dims, other keys), then the
            // waves through LDS.
#pragma unroll
            for (int sh = LPR; sh <= 32; sh <<= 1) {
                // The two states of lanes l and l ^ sh (a DPP row rotation by 8, or
                // v_permlane16/32_swap); the merge is symmetric in them.
                auto sw = [&](float v) {
                    return sh == 8 ? LanePair{v, dpp_mov<0x128>(v)} : sh == 16 ? swap16(v) : swap32(v);
                };
                const LanePair pm = sw(m), pl = sw(lsum);
                const float mn = fmaxf(pm.a, pm.b);
                const float fa = pm.a == -INFINITY ? 0.f : exp2f(pm.a - mn);
                const float fb = pm.b == -INFINITY ? 0.f : exp2f(pm.b - mn);
                lsum = pl.a * fa + pl.b * fb;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const LanePair po = sw(o[e]);
                    o[e] = po.a * fa + po.b * fb;
                }
                m = mn;
            }
            if (lane == 0) {
                s_am[wave] = m;
                s_al[wave] = lsum;
            }
            if (ag == 0 && !padl) {
#pragma unroll
                for (int e = 0; e < 8; ++e) sO[wave * HD + lr * 8 + e] = o[e];
            }
            if (!all_ok(ok, &s_fail)) return;
            DPROG_STAMP(1 + l * 8 + 5);
            // The split's state over its 8 waves: o_d (d = tid), M, L.
            float M = -INFINITY, L = 0.f, acc = 0.f;
            if (tid < HD + 2) {
#pragma unroll
                for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_am[w]);
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float fw = s_am[w] == -INFINITY ? 0.f : exp2f(s_am[w] - M);
                    L += s_al[w] * fw;
                    if (tid < HD) acc += sO[w * HD + tid] * fw;
                }
            }
            bool mok = true;
            if (NS > 1 && s > 0) {
                if (tid < HD + 2) {
                    const float v = tid < HD ? acc : (tid == HD ? M : L);
                    const uint64_t w = (uint64_t)__float_as_uint(v) | ((uint64_t)tag << 32);
                    __hip_atomic_store(f_part + (size_t)(h * NS + s) * kPartWords + tid, w,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            } else if (NS > 1) {
                // Split 0 folds in splits 1 .. NS-1: thread d < HD waits for word d of
                // every sibling, thread j - 1 (j < NS) also for sibling j's max and sum,
                // which it passes on through LDS. Each round requests every word still
                // missing at once, with buffer loads that never branch (a word already
                // held, or not wanted, takes an offset past the buffer and touches no
                // memory), so a round costs one round trip. Reloads behind per-word
                // branches were each followed by a wait for that load, one round trip
                // per sibling per round.
                const int mj = tid + 1;  // sibling whose max / sum this thread fetches
                const uint32_t pbytes = (uint32_t)(NS * kPartWords * 8);
                const __amdgpu_buffer_rsrc_t rp = rsrc(f_part + (size_t)h * NS * kPartWords, pbytes);
                float vo[kNSMax];
                unsigned pend = 0;
#pragma unroll
                for (int j = 1; j < kNSMax; ++j) {
                    vo[j] = 0.f;
                    if (tid < HD && j < NS) pend |= 1u << j;
                }
                if (tid < HD && mj < NS) pend |= 1u;
                const uint32_t off_m = (uint32_t)((mj * kPartWords + HD) * 8);
                uint2 wv[kNSMax], wm, wl;
                auto request = [&]() {
#pragma unroll
                    for (int j = 1; j < kNSMax; ++j)
                        wv[j] = ld64<kSC1>(rp, ((pend >> j) & 1u) ? (uint32_t)((j * kPartWords + tid) * 8)
                                                                  : pbytes);
                    wm = ld64<kSC1>(rp, (pend & 1u) ? off_m : pbytes);
                    wl = ld64<kSC1>(rp, (pend & 1u) ? off_m + 8u : pbytes);
                };
                request();
                unsigned long long t0 = 0;
                for (unsigned it = 0; pend; ++it) {
#pragma unroll
                    for (int j = 1; j < kNSMax; ++j)
                        if (((pend >> j) & 1u) && wv[j].y == tag) {
                            vo[j] = __uint_as_float(wv[j].x);
                            pend &= ~(1u << j);
                        }
                    if ((pend & 1u) && wm.y == tag && wl.y == tag) {
                        s_pm[mj] = __uint_as_float(wm.x);
                        s_pl[mj] = __uint_as_float(wl.x);
                        pend &= ~1u;
                    }
                    if (!pend) break;
                    if (!keep_waiting(f, it, t0)) {
                        mok = false;
                        break;
                    }
                    request();
                }
                if (!all_ok(mok, &s_fail)) return;
                DPROG_STAMP(1 + l * 8 + 6);
                if (tid < HD) {
                    float Mt = M;
                    for (int j = 1; j < NS; ++j) Mt = fmaxf(Mt, s_pm[j]);
                    const float f0 = M == -INFINITY ? 0.f : exp2f(M - Mt);
                    float num = acc * f0, den = L * f0;
#pragma unroll
                    for (int j = 1; j < kNSMax; ++j)
                        if (j < NS) {
                            const float fw = s_pm[j] == -INFINITY ? 0.f : exp2f(s_pm[j] - Mt);
                            num += vo[j] * fw;
                            den += s_pl[j] * fw;
                        }
                    put(rsrc(f_att, (uint32_t)HO * 4), h * HD + tid, den > 0.f ? num / den : 0.f, tag);
                }
            } else if (tid < HD) {
                put(rsrc(f_att, (uint32_t)HO * 4), h * HD + tid, L > 0.f ? acc / L : 0.f, tag);
            }
            // This split's K/V rows are consumed: the next layer's go to LDS now, once
            // this wave's output stores have completed (requests queued behind a
            // prefetch of the K/V rows would reach the consumers later).
            __builtin_amdgcn_s_waitcnt(0);
            DPROG_STAMP(1 + l * 8 + 3);
            if (l + 1 < p.L) kv_fetch(s_layers[l + 1]);
            if (!all_ok(mok, &s_fail)) return;
        }
        // The final norm's residual: the last layer's post-attention residual,
        // published by workgroup 0.
        {
            const int units = D / 8;
            const uint32_t bytes = (uint32_t)D * 4u;
            const uint32_t offr[1] = {tid < units ? (uint32_t)tid * 32u : bytes};
            uint4 rv[1];
            const bool rok = poll_units<1>(rsrc(f_res, bytes), offr, tid < units ? 1u : 0u, f, rv);
            if (rok && tid < units) sR[tid] = rv[0];
            if (!all_ok(rok, &s_fail)) return;
        }
    } else {
        // --------------------------------------------------- projection workgroups
        // Rows are dealt to workgroups [0, NC) in contiguous ranges (a phase's outputs
        // of one workgroup are then one block of the vector, written by one store
        // instruction: lines written piecewise by many CUs cost several microseconds
        // to settle), and within a workgroup to its waves.
        const int ng_q = (NQ + 3) / 4, ng_o = (D + 3) / 4, ng_gu = (2 * I + 3) / 4;
        const int gq = p.gq, go = p.go, ggu = p.ggu, gd = p.gd;
        const int q_g = wave < gq ? wg * gq + wave : ng_q;  // QKV group
        // A second QKV group per wave when the share exceeds one group per wave: read
        // into registers at the end of the previous layer's A (or before the first).
        const int q_g2 = wave + kWaves < gq ? wg * gq + wave + kWaves : ng_q;
        const int o_g = wave < go ? wg * go + wave : ng_o;  // o_proj group
        const int d_row = wave < gd ? wg * gd + wave : D;   // down row
        // A second down row per wave when the share exceeds one row per wave: read
        // into registers at the end of D (its wait overlaps the D -> E hop).
        const int d_row2 = wave + kWaves < gd ? wg * gd + wave + kWaves : D;
        uint32_t sq[1][CPLD], so[CPLD], sg[kGu][CPLD], sd[1][kIChunksPerLane];
        Rows<kIChunksPerLane> dr2;
        // With one gate/up group per wave in LDS (wide rows), the wave's next two
        // groups and its second down row are read into registers at the end of A,
        // their wait overlapping the attention phase instead of sitting inside D or
        // before E (requested at the end of C or D, loads delayed the next poll,
        // which completes in order behind them).
        constexpr bool kGuReg = kGu <= 2;
        Rows<CPLD> gx, gx2, qx;
        auto qkv2_load = [&](const OrtmiDecoderLayer& lz) {
            const int li = opaque(threadIdx.x & 63) & 15, gp = (threadIdx.x & 63) >> 4;
            load_rows<16, CPLD>(qx, weight_ref(lz.qkv_weight, lz.qkv_scales, NQ, CD),
                                q_g2 < ng_q ? 4 * q_g2 + gp : NQ, li);
        };
        // Weights are requested two phases ahead of their use, into slot ranges no
        // phase in between reads: end of A -> gate/up, end of C -> down, end of D ->
        // next QKV, end of E -> next o_proj (region_lo).
        {
            const WeightRef wr = weight_ref(s_layers[0].qkv_weight, s_layers[0].qkv_scales, NQ, CD);
            fetch_rows<16, CPLD>(wr, q_g < ng_q ? 4 * q_g + grp : NQ, li16, wreg, sq[0]);
            const WeightRef wo = weight_ref(s_layers[0].o_weight, s_layers[0].o_scales, D, CO);
            fetch_rows<16, CPLD>(wo, o_g < ng_o ? 4 * o_g + grp : D, li16, wreg + kLo * 64, so);
            if (gq > kWaves) qkv2_load(s_layers[0]);
        }
        const uint32_t* in_dout = nullptr;
        for (int l = 0; l < p.L; ++l) {
            const OrtmiDecoderLayer& ly = s_layers[l];
            // Lane-derived indices, recomputed per layer rather than held across it.
            const int lane = opaque(threadIdx.x & 63);
            const int li16 = lane & 15, grp = lane >> 4;
            auto qkv_fetch = [&](const OrtmiDecoderLayer& lz) {
                const WeightRef wr = weight_ref(lz.qkv_weight, lz.qkv_scales, NQ, CD);
                fetch_rows<16, CPLD>(wr, q_g < ng_q ? 4 * q_g + grp : NQ, li16, wreg, sq[0]);
            };
            auto o_fetch = [&](const OrtmiDecoderLayer& lz) {
                const WeightRef wr = weight_ref(lz.o_weight, lz.o_scales, D, CO);
                fetch_rows<16, CPLD>(wr, o_g < ng_o ? 4 * o_g + grp : D, li16, wreg + kLo * 64, so);
            };
            auto gu_fetch = [&]() {
                const WeightRef wr = weight_ref(ly.gate_up_weight, ly.gate_up_scales, 2 * I, CD);
#pragma unroll
                for (int k = 0; k < kGu; ++k) {
                    const int lg = wave + k * kWaves;
                    const int g = lg < ggu ? wg * ggu + lg : ng_gu;
                    fetch_rows<16, CPLD>(wr, g < ng_gu ? 4 * g + grp : 2 * I, li16,
                                         wreg + k * CPLD * 64, sg[k]);
                }
            };
            auto down_fetch = [&]() {
                const WeightRef wr = weight_ref(ly.down_weight, ly.down_scales, D, CI);
                fetch_rows<64, kIChunksPerLane>(wr, d_row, lane, wreg + kLo * 64, sd[0]);
            };
            uint32_t* f_qkv = p.flow + (size_t)l * p.flow_stride;
            uint32_t* f_att = f_qkv + NQ;
            uint32_t* f_y = f_att + HO;
            uint32_t* f_act = f_y + D;
            uint32_t* f_dout = f_act + I;

            // Phase A: input norm (+ residual), merged QKV GEMV.
            if (!norm_poll(in_dout, p.embed + id * D, l > 0, static_cast<const half_t*>(ly.ln1_gamma),
                           ly.ln1_epsilon, D, sR, sA0, sSum0, sRed, f, &s_fail))
                return;
            DPROG_STAMP(1 + l * 8);
            {
                __builtin_amdgcn_s_waitcnt(0);
                if (gq > kWaves) {
                    // Both QKV groups of the wave in one pass over the activations.
                    float qa[2];
                    const Rows<CPLD>* const rg[1] = {&qx};
                    rows_dot_multi<16, CPLD, 1, 1>(wreg, sq, rg, sA0, sSum0, CD, li16, qa);
                    const float v = group_sum<16>(qa[0]), v2 = group_sum<16>(qa[1]);
                    if (li16 == 0 && wave < gq) s_out[wave * 4 + grp] = v;
                    if (li16 == 0 && wave + kWaves < gq) s_out[(wave + kWaves) * 4 + grp] = v2;
                } else {
                    const float v = group_sum<16>(row_dot<16, CPLD>(wreg, sq[0], sA0, sSum0, CD, li16));
                    if (li16 == 0 && wave < gq) s_out[wave * 4 + grp] = v;
                }
                __syncthreads();
                if (tid < 4 * gq && 4 * wg * gq + tid < NQ)
                    put(rsrc(f_qkv, (uint32_t)NQ * 4), 4 * wg * gq + tid, s_out[tid], tag);
                DPROG_STAMP(1 + l * 8 + 1);
                wait_lds();
                gu_fetch();
                if (gq > kWaves && l + 1 < p.L) qkv2_load(s_layers[l + 1]);
                if constexpr (kGuReg) {
                    const WeightRef wr = weight_ref(ly.gate_up_weight, ly.gate_up_scales, 2 * I, CD);
                    const int lg = wave + kGu * kWaves, lg2 = lg + kWaves;
                    const int g = lg < ggu ? wg * ggu + lg : ng_gu;
                    const int g2 = lg2 < ggu ? wg * ggu + lg2 : ng_gu;
                    load_rows<16, CPLD>(gx, wr, g < ng_gu ? 4 * g + grp : 2 * I, li16);
                    load_rows<16, CPLD>(gx2, wr, g2 < ng_gu ? 4 * g2 + grp : 2 * I, li16);
                    if (gd > kWaves)
                        load_rows<64, kIChunksPerLane>(
                            dr2, weight_ref(ly.down_weight, ly.down_scales, D, CI), d_row2, lane);
                }
            }

            // Phase C: o_proj GEMV over the attention output.
            if (!stage_poll(f_att, HO, sA1, sSum1, f, &s_fail)) return;
            DPROG_STAMP(1 + l * 8 + 2);
            {
                __builtin_amdgcn_s_waitcnt(0);
                const float v = group_sum<16>(row_dot<16, CPLD>(wreg + kLo * 64, so, sA1, sSum1, CO, li16));
                if (li16 == 0 && wave < go) s_out[wave * 4 + grp] = v;
                __syncthreads();
                if (tid < 4 * go && 4 * wg * go + tid < D)
                    put(rsrc(f_y, (uint32_t)D * 4), 4 * wg * go + tid, s_out[tid], tag);
                DPROG_STAMP(1 + l * 8 + 3);
                wait_lds();
                down_fetch();
            }

            // Phase D: residual + post-attention norm, gate/up GEMV with SwiGLU.
            if (!norm_poll(f_y, nullptr, true, static_cast<const half_t*>(ly.ln2_gamma), ly.ln2_epsilon,
                           D, sR, sA0, sSum0, sRed, f, &s_fail))
                return;
            DPROG_STAMP(1 + l * 8 + 4);
            if (l + 1 == p.L && wg == 0) {
                // The final norm's residual, for the attention workgroups.
                for (int u = tid; u < D / 8; u += kThreads) {
                    const uint4 r = sR[u];
                    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
                    const __amdgpu_buffer_rsrc_t rr = rsrc(f_res, (uint32_t)D * 4);
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        __builtin_amdgcn_raw_buffer_store_b32(((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) | (tag << 16),
                                                              rr, (uint32_t)(u * 8 + e) * 4u, 0, kSC1);
                }
            }
            {
                const __amdgpu_buffer_rsrc_t ra = rsrc(f_act, (uint32_t)I * 4);
                // Local group lg of this workgroup: rows 4g .. 4g+3 (gate, up, gate, up),
                // g = wg * ggu + lg, giving pairs 2g and 2g + 1 (local 2lg, 2lg + 1).
                auto gu_out = [&](float v, int lg) {
                    v = group_sum<16>(v);
                    const float other = __shfl_xor(v, 16, 64);  // gate (even group) <-> up (odd)
                    const int g = wg * ggu + lg;
                    if (lg < ggu && g < ng_gu && li16 == 0 && (grp & 1) == 0) {
                        const float gv = r16(v), up = r16(other);
                        const float sig = r16(1.0f / (1.0f + __expf(-gv)));
                        s_out[2 * lg + (grp >> 1)] = r16(r16(gv * sig) * up);
                    }
                };
                __builtin_amdgcn_s_waitcnt(0);
                // The LDS groups (and, with wide rows, the two register groups) in
                // one pass over the activation chunks.
                int lg0 = wave + kGu * kWaves;
                if constexpr (kGuReg) {
                    float gacc[kGu + 2];
                    const Rows<CPLD>* const rg[2] = {&gx, &gx2};
                    rows_dot_multi<16, CPLD, kGu, 2>(wreg, sg, rg, sA0, sSum0, CD, li16, gacc);
#pragma unroll
                    for (int k = 0; k < kGu; ++k) gu_out(gacc[k], wave + k * kWaves);
                    gu_out(gacc[kGu], lg0);
                    gu_out(gacc[kGu + 1], lg0 + kWaves);
                    lg0 += 2 * kWaves;
                } else {
                    float gacc[kGu];
                    const Rows<CPLD>* const rg[1] = {nullptr};
                    rows_dot_multi<16, CPLD, kGu, 0>(wreg, sg, rg, sA0, sSum0, CD, li16, gacc);
#pragma unroll
                    for (int k = 0; k < kGu; ++k) gu_out(gacc[k], wave + k * kWaves);
                }
                const WeightRef wr = weight_ref(ly.gate_up_weight, ly.gate_up_scales, 2 * I, CD);
                for (int lg = lg0; lg < ggu; lg += kWaves) {
                    const int g = wg * ggu + lg;
                    Rows<CPLD> r;
                    load_rows<16, CPLD>(r, wr, g < ng_gu ? 4 * g + grp : 2 * I, li16);
                    gu_out(rows_dot<16, CPLD>(r, sA0, sSum0, CD, li16), lg);
                }
                __syncthreads();
                if (tid < 2 * ggu && 2 * wg * ggu + tid < I)
                    put(ra, 2 * wg * ggu + tid, s_out[tid], tag);
                DPROG_STAMP(1 + l * 8 + 5);
                wait_lds();
                if (l + 1 < p.L) qkv_fetch(s_layers[l + 1]);
                if (!kGuReg && gd > kWaves)
                    load_rows<64, kIChunksPerLane>(
                        dr2, weight_ref(ly.down_weight, ly.down_scales, D, CI), d_row2, lane);
            }

            // Phase E: down GEMV (K = I).
            if (!stage_poll(f_act, I, sA1, sSum1, f, &s_fail)) return;
            DPROG_STAMP(1 + l * 8 + 6);
            {
                __builtin_amdgcn_s_waitcnt(0);
                if (gd > kWaves) {
                    // Both down rows of the wave in one pass over the activations.
                    float da[2];
                    const Rows<kIChunksPerLane>* const rg[1] = {&dr2};
                    rows_dot_multi<64, kIChunksPerLane, 1, 1>(wreg + kLo * 64, sd, rg, sA1, sSum1, CI, lane, da);
                    const float v = wave_sum(da[0]), v2 = wave_sum(da[1]);
                    if (lane == 0 && wave < gd) s_out[wave] = v;
                    if (lane == 0 && wave + kWaves < gd) s_out[wave + kWaves] = v2;
                } else {
                    const float v =
                        wave_sum(row_dot<64, kIChunksPerLane>(wreg + kLo * 64, sd[0], sA1, sSum1, CI, lane));
                    if (lane == 0 && wave < gd) s_out[wave] = v;
                }
                __syncthreads();
                if (tid < gd && wg * gd + tid < D)
                    put(rsrc(f_dout, (uint32_t)D * 4), wg * gd + tid, s_out[tid], tag);
                DPROG_STAMP(1 + l * 8 + 7);
                wait_lds();
                if (l + 1 < p.L) o_fetch(s_layers[l + 1]);
            }
            in_dout = f_dout;
        }
    }

    // Phase F: final norm, lm_head GEMV (logits), argmax. The first lm_head rows are
    // requested before the wait for the last down output.
    constexpr int kRing = CPLD <= 4 ? 4 : 2;
    const int lm_ng = (p.V + 3) / 4;
    const WeightRef lw = weight_ref(p.lm_w, p.lm_s, p.V, CD);
    Rows<CPLD> ring[kRing];
#pragma unroll
    for (int r = 0; r < kRing; ++r) {
        const int g = gw + r * TW;
        load_rows<16, CPLD>(ring[r], lw, g < lm_ng ? 4 * g + grp : p.V, li16);
    }
    if (!norm_poll(prev_dout, nullptr, true, p.final_gamma, p.final_eps, D, sR, sA0, sSum0, sRed,
                   f, &s_fail))
        return;
    DPROG_STAMP(1 + p.L * 8);
    float best = -INFINITY;
    int bi = -1;
    for (int k = 0;; k += kRing) {
        bool done = false;
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            const int g = gw + (k + r) * TW;
            if (g >= lm_ng) {
                done = true;
                break;
            }
            const float v = group_sum<16>(rows_dot<16, CPLD>(ring[r], sA0, sSum0, CD, li16));
            const int gn = g + kRing * TW;
            load_rows<16, CPLD>(ring[r], lw, gn < lm_ng ? 4 * gn + grp : p.V, li16);
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
    DPROG_STAMP(2 + p.L * 8);
    // Reduce (value, index) over the workgroup, publish one tagged record.
    arg_wave(best, bi);
    if (lane == 0) {
        s_arg_v[wave] = best;
        s_arg_i[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w = 0; w < kWaves; ++w) arg_take(best, bi, s_arg_v[w], s_arg_i[w]);
        const uint64_t rec = (uint64_t)(uint32_t)bi | ((uint64_t)f2h(best) << 32) |
                             ((uint64_t)tag << 48);
        __hip_atomic_store(p.argp + wg, rec, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wg != 0) return;
    best = -INFINITY;
    bi = -1;
    bool ok = true;
    for (int w0 = 0; w0 < nwg; w0 += kThreads) {
        const int w = w0 + tid;
        if (w >= nwg) continue;
        uint64_t rec = 0;
        unsigned long long t0 = 0;
        for (unsigned it = 0;; ++it) {
            rec = __hip_atomic_load(p.argp + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)(rec >> 48) == tag) break;
            if (!keep_waiting(f, it, t0)) {
                ok = false;
                break;
            }
        }
        if (!ok) break;
        arg_take(best, bi, h2f((uint32_t)(rec >> 32) & 0xFFFFu), (int)(uint32_t)rec);
    }
    arg_wave(best, bi);
    if (lane == 0) {
        s_arg_v[wave] = best;
        s_arg_i[wave] = bi;
    }
    if (!all_ok(ok, &s_fail)) return;
    if (tid == 0) {
        for (int w = 0; w < kWaves; ++w) arg_take(best, bi, s_arg_v[w], s_arg_i[w]);
        *p.next_id = bi < 0 ? 0 : bi;
        store_status(p.status, bad_id ? 2 : 0);
        DPROG_STAMP(kStampSlots - 2);  // greedy id written (workgroup 0)
    }
}

}  // namespace dprog
}  // namespace ortmi

using namespace ortmi;

namespace {

struct StepShape {
    size_t ctl, flow, part, argp, total;
    uint32_t flow_stride;
};

// Rows of each projection phase per projection workgroup (groups of 4 rows for
// QKV, o_proj and gate/up; single rows for down) with `nc` projection workgroups.
struct Shares {
    int gq, go, ggu, gd;
    bool fit() const {
        return gq <= 2 * dprog::kWaves && go <= dprog::kWaves && gd <= 2 * dprog::kWaves &&
               2 * ggu <= 64;
    }
};
Shares step_shares(const OrtmiDecoderDims* d, int nc) {
    const int nq = (d->num_heads + 2 * d->kv_num_heads) * d->head_size;
    Shares s;
    s.gq = ((nq + 3) / 4 + nc - 1) / nc;
    s.go = ((d->hidden + 3) / 4 + nc - 1) / nc;
    s.ggu = ((2 * d->intermediate + 3) / 4 + nc - 1) / nc;
    s.gd = (d->hidden + nc - 1) / nc;
    return s;
}

// Key splits per attention head: about 160 keys each (their K/V rows fit one
// workgroup's LDS), while at least half the workgroups stay on the projections
// and each projection workgroup's share of rows fits its waves.
int step_splits(const OrtmiDecoderDims* d, int nwg) {
    int ns = (d->kv_capacity + 159) / 160;
    ns = ns < 1 ? 1 : (ns > dprog::kNSMax ? dprog::kNSMax : ns);
    while (ns > 1 && (nwg - d->num_heads * ns < nwg / 2 ||
                      !step_shares(d, nwg - d->num_heads * ns).fit()))
        --ns;
    return ns;
}

StepShape step_layout(const OrtmiDecoderDims* d, int nwg) {
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    StepShape s{};
    const size_t words = (size_t)(d->num_heads + 2 * d->kv_num_heads) * d->head_size +
                         (size_t)d->num_heads * d->head_size + 2 * (size_t)d->hidden +
                         (size_t)d->intermediate;
    s.flow_stride = (uint32_t)((words + 63) & ~(size_t)63);
    size_t off = 0;
    s.ctl = off;
    off += dprog::kCtlBytes;
    s.flow = off;  // per layer, then the final norm's residual [hidden]
    off += al(((size_t)std::max(d->layers, 0) * s.flow_stride + (size_t)d->hidden) * 4);
    s.part = off;
    off += al((size_t)std::max(d->layers, 0) * d->num_heads * step_splits(d, nwg) *
              dprog::kPartWords * 8);
    s.argp = off;
    off += al((size_t)nwg * 8);
    s.total = off;
    return s;
}

int program_grid() {
    const int cus = device_cu_count();
    return cus - cus % kXcds;
}

}  // namespace

#ifdef ORTMI_DPROG_STAMPS
// The stamps of the last launch: `rows` workgroup rows of kStampSlots 64-bit clock
// values (100 MHz), copied to host memory after the device has finished.
extern "C" int ortmi_decoder_decode_step_stamps(unsigned long long* host, int rows) {
    if (!host || rows < 1 || rows > 1024) return fail(ORTMI_E_INVALID, "stamps: bad rows");
    const hipError_t e = hipMemcpyFromSymbol(host, HIP_SYMBOL(dprog::g_stamps),
                                             (size_t)rows * dprog::kStampSlots * 8, 0,
                                             hipMemcpyDeviceToHost);
    return e == hipSuccess ? ORTMI_OK : fail(ORTMI_E_HIP, hipGetErrorString(e));
}
#endif

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
    ORTMI_REQUIRE(d.layers >= 1 && d.layers <= dprog::kMaxLayers, "decoder step: 1 to 64 layers");
    ORTMI_REQUIRE(d.head_size == 128 || d.head_size == 96 || d.head_size == 64,
                  "decoder step: head size 64, 96 or 128");
    ORTMI_REQUIRE(d.num_heads > 0 && d.kv_num_heads > 0 && d.num_heads % d.kv_num_heads == 0 &&
                      d.num_heads / d.kv_num_heads <= dprog::kGMax,
                  "decoder step: at most 8 query heads per KV head");
    ORTMI_REQUIRE(d.hidden % 32 == 0 && d.hidden <= 3072, "decoder step: hidden % 32 == 0, <= 3072");
    ORTMI_REQUIRE((d.num_heads * d.head_size) % 32 == 0 && d.num_heads * d.head_size <= 3072,
                  "decoder step: num_heads * head_size % 32 == 0, <= 3072");
    ORTMI_REQUIRE(d.intermediate % 32 == 0 && d.intermediate <= 64 * 32 * dprog::kIChunksPerLane,
                  "decoder step: intermediate % 32 == 0, <= 10240");
    ORTMI_REQUIRE(d.vocab > 0 && embed_rows > 0 && d.kv_capacity > 0, "decoder step: bad sizes");
    ORTMI_REQUIRE(d.rotary_half == 0 || (d.rotary_half % 8 == 0 && 2 * d.rotary_half <= d.head_size &&
                                          cos_cache && sin_cache && d.max_position > 0),
                  "decoder step: rotary half must be a multiple of 8, at most head_size / 2");
    ORTMI_REQUIRE(d.rotary_interleaved == 0, "decoder step: interleaved rotary is not supported");
    const int nwg = program_grid();
    ORTMI_REQUIRE(nwg >= 4 * d.num_heads && nwg >= kXcds,
                  "decoder step: needs at least 4 compute units per query head");
    const int ns = step_splits(dims, nwg);
    const int nc = nwg - d.num_heads * ns;
    const Shares sh = step_shares(dims, nc);
    const int gq = sh.gq, go = sh.go, ggu = sh.ggu, gd = sh.gd;
    ORTMI_REQUIRE(sh.fit(), "decoder step: projection rows exceed the per-workgroup share");
    ORTMI_REQUIRE((int64_t)d.kv_num_heads * d.kv_capacity * d.head_size * 2 < (int64_t)INT32_MAX &&
                      (int64_t)d.vocab * d.hidden / 2 < (int64_t)INT32_MAX,
                  "decoder step: a cache or the lm_head exceeds 2 GiB");
    const StepShape s = step_layout(dims, nwg);
    if (workspace_bytes < s.total)
        return fail(ORTMI_E_WORKSPACE, "decoder step: workspace too small");
    ORTMI_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0 &&
                      (reinterpret_cast<uintptr_t>(embed) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(final_gamma) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(cos_cache) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(sin_cache) & 15) == 0 &&
                      (reinterpret_cast<uintptr_t>(layers) & 3) == 0,
                  "decoder step: workspace, embedding, gamma and cos/sin must be 16-byte aligned");

    char* ws = static_cast<char*>(workspace);
    dprog::Params p{};
    p.layers = layers;
    p.L = d.layers;
    p.D = d.hidden;
    p.H = d.num_heads;
    p.KV = d.kv_num_heads;
    p.G = d.num_heads / d.kv_num_heads;
    p.I = d.intermediate;
    p.V = d.vocab;
    p.cap = d.kv_capacity;
    p.max_pos = d.max_position;
    p.half = d.rotary_half;
    p.nwg = nwg;
    p.gq = gq;
    p.go = go;
    p.ggu = ggu;
    p.gd = gd;
    p.nc = nc;
    p.ns = ns;
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
    p.flow = reinterpret_cast<uint32_t*>(ws + s.flow);
    p.flow_stride = s.flow_stride;
    p.part = reinterpret_cast<uint64_t*>(ws + s.part);
    p.argp = reinterpret_cast<uint64_t*>(ws + s.argp);

    // Chunks of 32 codes per lane for the K = hidden and K = H * head rows (16 lanes
    // per row): 3, 4 or 6.
    const int kmax = std::max(d.hidden, d.num_heads * d.head_size);
    const int cpld = kmax <= 1536 ? 3 : kmax <= 2048 ? 4 : 6;
    const void* fn =
        d.head_size == 128
            ? (cpld == 3   ? (const void*)dprog::decode_program_kernel<128, 3>
               : cpld == 4 ? (const void*)dprog::decode_program_kernel<128, 4>
                           : (const void*)dprog::decode_program_kernel<128, 6>)
        : d.head_size == 96
            ? (cpld == 3   ? (const void*)dprog::decode_program_kernel<96, 3>
               : cpld == 4 ? (const void*)dprog::decode_program_kernel<96, 4>
                           : (const void*)dprog::decode_program_kernel<96, 6>)
            : (cpld == 3   ? (const void*)dprog::decode_program_kernel<64, 3>
               : cpld == 4 ? (const void*)dprog::decode_program_kernel<64, 4>
                           : (const void*)dprog::decode_program_kernel<64, 6>);
    const int ho = d.num_heads * d.head_size;
    const size_t lds = ((size_t)dprog::kWaves * dprog::region_slots(cpld) * 64 + d.hidden / 8 +
                        std::max(ho, d.intermediate) / 8 + d.hidden / 8) * 16 +
                       ((size_t)dprog::kWaves * d.head_size + d.hidden / 32 +
                        std::max(ho, d.intermediate) / 32) * 4;
    // The fit check is made once per (device, kernel, LDS size).
    static std::mutex fit_mu;
    static std::map<std::tuple<int, const void*, size_t>, bool> fits;
    int dev = 0;
    (void)hipGetDevice(&dev);
    bool fit;
    {
        std::lock_guard<std::mutex> lock(fit_mu);
        auto it = fits.find({dev, fn, lds});
        if (it == fits.end()) {
            int per_cu = 0;
            fit = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, dprog::kThreads, lds) ==
                      hipSuccess && per_cu >= 1;
            (void)hipGetLastError();
            fits[{dev, fn, lds}] = fit;
        } else {
            fit = it->second;
        }
    }
    if (!fit) return fail(ORTMI_E_INVALID, "decoder step: the program does not fit one workgroup per CU");
    // One workgroup per CU, at most one fits per CU: with the device otherwise idle a
    // plain launch makes every workgroup resident at once, and costs about 30 us less
    // per step than a cooperative launch, which guarantees it. Either way every wait
    // inside is bounded, so a workgroup that cannot start (another kernel holds its
    // CU) makes the launch stop with status 1 rather than hang; the caller then runs
    // the step op by op and can ask for cooperative launches from then on.
    void* args[] = {&p};
    const hipError_t e =
        d.cooperative ? hipLaunchCooperativeKernel(fn, dim3(nwg), dim3(dprog::kThreads), args,
                                                   (unsigned)lds, as_stream(stream))
                      : hipLaunchKernel(fn, dim3(nwg), dim3(dprog::kThreads), args, (size_t)lds,
                                        as_stream(stream));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(ORTMI_E_HIP, std::string("decoder step: launch: ") + hipGetErrorString(e));
    }
    return ORTMI_OK;
}
