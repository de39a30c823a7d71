// GroupQueryAttention for the forms the fused fp16/bf16 kernels do not take:
// fp32 tensors, per-head QK RMS-norm (inputs 14/15), an additive attention_bias
// (input 10) and head sizes other than 64/128 (multiples of 16 up to 256).
//
// Two kernels:
//  - gqa_ex_prep_kernel: one wave per (token, head) vector. Q heads: optional
//    RMS-norm, optional RoPE at position valid_past + s, each step rounded to the
//    op dtype as the reference materialises it (rust/src/ops/attention.rs:663-708),
//    written to an fp32 workspace. K heads: the same, written to present_key at row
//    valid_past + s. V heads: copied to present_value.
//  - gqa_ex_attn_kernel: one workgroup of 16 teams x 16 lanes per (token, query
//    head). Team t scores keys t, t+16, ... (a 16-lane dot product reduced inside a
//    DPP row), adds the bias, and keeps an online softmax; the 16 team states are
//    merged through LDS. Causal: query s attends keys [0, valid_past + s].
// The KV contract (shared buffer vs growing, attention.rs:636-651) is that of
// ortmi_group_query_attention.
//
// The sliding-window cache (sliding_window_cache = 1, attention.rs:725-880) adds
// two: gqa_sw_attn_kernel (the same teams, keys read from the cached rows and the
// new rows of the query's window) and gqa_sw_present_kernel (the compacted
// present: the last cache_end(length) rows, zeros after). The prep kernel then
// takes per-sequence positions from seqlens_k and writes the new K/V rows to a
// workspace instead of present.

#include <algorithm>
#include <cmath>

#include "common.h"

namespace ortmi {
namespace {

constexpr int kTeamLanes = 16;
constexpr int kTeams = 16;
constexpr int kMaxHead = 256;
constexpr int kMaxPerLane = kMaxHead / kTeamLanes;  // 16

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Copies the first `rows` rows of every [cap, row_words] head block of src into
// the [dst_cap, row_words] block of dst (32-bit words).
__global__ __launch_bounds__(256) void kv_rows_copy_kernel(const uint32_t* __restrict__ src,
                                                           uint32_t* __restrict__ dst,
                                                           int64_t src_cap, int64_t dst_cap,
                                                           int64_t rows, int row_words,
                                                           int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t per_head = rows * row_words;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t bh = i / per_head;
        const int64_t rem = i - bh * per_head;
        dst[bh * dst_cap * row_words + rem] = src[bh * src_cap * row_words + rem];
    }
}

// grid (B*S, H + 2*KV), block 64 (one wave per head vector of hd <= 256 dims;
// lane l holds dims l, l+64, l+128, l+192).
template <typename T>
__global__ __launch_bounds__(64) void gqa_ex_prep_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v, int64_t q_stride,
    int64_t kv_stride, const T* __restrict__ cos_c, const T* __restrict__ sin_c, int half,
    int interleaved, const T* __restrict__ qw, const T* __restrict__ kw, float eps,
    float* __restrict__ qf, T* __restrict__ pk, T* __restrict__ pv, int S, int H, int KV, int hd,
    int64_t pcap, int vp, const int* __restrict__ seqlens, int max_pos) {
    __shared__ float sx[kMaxHead];
    const int bs = blockIdx.x;
    const int b = bs / S, s = bs % S;
    const int head = blockIdx.y;
    const int lane = threadIdx.x;
    // Rotary position and destination row: valid_past + s for the dense contracts;
    // with seqlens (the sliding-window cache) the sequence's own past length
    // max(seqlens_k + 1 - S, 0) + s, clamped to the cos/sin rows, and row s of the
    // [B, KV, S, hd] new-row workspace.
    int64_t pos = vp + s, row = vp + s;
    if (seqlens) {
        pos = min(max((int64_t)seqlens[b] + 1 - S, (int64_t)0) + s, (int64_t)max(max_pos - 1, 0));
        row = s;
    }
    if (head >= H + KV) {  // V head: copied as is
        const int kh = head - H - KV;
        const T* src = v + (int64_t)bs * kv_stride + (int64_t)kh * hd;
        T* dst = pv + (((int64_t)b * KV + kh) * pcap + row) * hd;
        for (int d = lane; d < hd; d += 64) dst[d] = src[d];
        return;
    }
    const bool is_q = head < H;
    const int kh = head - H;
    const T* src = is_q ? q + (int64_t)bs * q_stride + (int64_t)head * hd
                        : k + (int64_t)bs * kv_stride + (int64_t)kh * hd;
    const T* w = is_q ? qw : kw;
    float x[4];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = lane + 64 * e;
        x[e] = d < hd ? to_f32(src[d]) : 0.f;
        ss += x[e] * x[e];
    }
    if (w) {  // QK-norm: y = x / sqrt(mean(x^2) + eps) * w, in the op dtype
        const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)hd + eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            if (d < hd) x[e] = round_to<T>(x[e] * inv * to_f32(w[d]));
        }
    }
    if (cos_c) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            if (d < hd) sx[d] = x[e];
        }
        __syncthreads();
        const T* crow = cos_c + pos * half;
        const T* srow = sin_c + pos * half;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            if (d >= 2 * half) continue;  // dims past the rotary span pass through
            if (interleaved) {
                const int i = d >> 1;
                const float c = to_f32(crow[i]), sn = to_f32(srow[i]);
                const float a = sx[d & ~1], bb = sx[d | 1];
                x[e] = round_to<T>((d & 1) ? bb * c + a * sn : a * c - bb * sn);
            } else {
                const int i = d < half ? d : d - half;
                const float c = to_f32(crow[i]), sn = to_f32(srow[i]);
                const float a = sx[i], bb = sx[i + half];
                x[e] = round_to<T>(d < half ? a * c - bb * sn : bb * c + a * sn);
            }
        }
    }
    if (is_q) {
        float* dst = qf + ((int64_t)bs * H + head) * hd;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            if (d < hd) dst[d] = x[e];
        }
    } else {
        T* dst = pk + (((int64_t)b * KV + kh) * pcap + row) * hd;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int d = lane + 64 * e;
            if (d < hd) dst[d] = from_f32<T>(x[e]);
        }
    }
}

// Rows a sliding-window cache of capacity cap holds after `length` tokens: once
// full it drops its oldest gap = cap - window + 1 rows at a time
// (attention.rs:736-745).
__device__ __forceinline__ int64_t sw_cache_end(int64_t length, int64_t cap, int64_t gap) {
    if (length <= cap) return length;
    return length - gap * ((length - cap + gap - 1) / gap);
}

// Sliding-window attention, grid (B*S*H), block 256 (the teams of
// gqa_ex_attn_kernel). The sequence's p = max(seqlens_k + 1 - S, 0) earlier
// tokens sit in cache rows [0, before), the last `before` of them; query s (position
// t = p + s) attends positions (t - window, t]: cached rows first, then the new
// rows (the workspace written by the prep kernel). Equal to the reference's
// working buffer with its causal window mask (attention.rs:786-839).
template <typename T>
__global__ __launch_bounds__(256) void gqa_sw_attn_kernel(
    const float* __restrict__ qf, const T* __restrict__ past_k, const T* __restrict__ past_v,
    const T* __restrict__ knew, const T* __restrict__ vnew, const int* __restrict__ seqlens,
    T* __restrict__ out, int S, int H, int KV, int hd, int cap, int window, float scale) {
    __shared__ float s_m[kTeams], s_l[kTeams];
    __shared__ float s_acc[kTeams][kMaxHead];
    const int row = blockIdx.x;  // (b*S + s)*H + h
    const int h = row % H;
    const int bs = row / H;
    const int b = bs / S, s = bs % S;
    const int kh = h / (H / KV);
    const int team = threadIdx.x / kTeamLanes;
    const int lt = threadIdx.x % kTeamLanes;
    const int E = hd / kTeamLanes;
    const int64_t p = max((int64_t)seqlens[b] + 1 - S, (int64_t)0);
    const int64_t before = sw_cache_end(p, cap, cap - window + 1);
    const int64_t t = p + s;
    const int64_t lo = max(t - window + 1, (int64_t)0);
    const int npast = (int)max(p - lo, (int64_t)0);      // cached keys, rows [before - npast, before)
    const int first_new = (int)max(lo - p, (int64_t)0);  // new keys [first_new, s]
    const int nk = npast + s - first_new + 1;
    const int64_t slab = (int64_t)b * KV + kh;
    const T* kc = past_k + (slab * cap + (before - npast)) * hd;
    const T* vc = past_v + (slab * cap + (before - npast)) * hd;
    const T* kn = knew + (slab * S + first_new) * hd;
    const T* vn = vnew + (slab * S + first_new) * hd;
    const float* qrow = qf + (int64_t)row * hd;

    float qv[kMaxPerLane], acc[kMaxPerLane];
#pragma unroll
    for (int e = 0; e < kMaxPerLane; ++e) {
        qv[e] = e < E ? qrow[lt + kTeamLanes * e] : 0.f;
        acc[e] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    for (int base = 0; base < nk; base += kTeams) {
        const int j = base + team;
        if (j >= nk) continue;  // uniform over the team's 16 lanes
        const bool cached = j < npast;
        const T* kr = cached ? kc + (int64_t)j * hd : kn + (int64_t)(j - npast) * hd;
        const T* vr = cached ? vc + (int64_t)j * hd : vn + (int64_t)(j - npast) * hd;
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < kMaxPerLane; ++e)
            if (e < E) dot += qv[e] * to_f32(kr[lt + kTeamLanes * e]);
        const float sc = group_sum<kTeamLanes>(dot) * scale;
        const float mn = fmaxf(m, sc);
        const float corr = __expf(m - mn);  // m = -inf -> 0
        const float pe = __expf(sc - mn);
        l = l * corr + pe;
#pragma unroll
        for (int e = 0; e < kMaxPerLane; ++e)
            if (e < E) acc[e] = acc[e] * corr + pe * to_f32(vr[lt + kTeamLanes * e]);
        m = mn;
    }
    if (lt == 0) {
        s_m[team] = m;
        s_l[team] = l;
    }
#pragma unroll
    for (int e = 0; e < kMaxPerLane; ++e)
        if (e < E) s_acc[team][lt + kTeamLanes * e] = acc[e];
    __syncthreads();
    float M = -INFINITY;
    for (int tm = 0; tm < kTeams; ++tm) M = fmaxf(M, s_m[tm]);
    T* orow = out + (int64_t)row * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float num = 0.f, den = 0.f;
        for (int tm = 0; tm < kTeams; ++tm) {
            if (s_m[tm] == -INFINITY) continue;
            const float wt = __expf(s_m[tm] - M);
            num += wt * s_acc[tm][d];
            den += wt * s_l[tm];
        }
        orow[d] = from_f32<T>(num / den);
    }
}

// The compacted present of a sliding-window cache, 32-bit words over
// [B, KV, cap, hd]: row r < after = cache_end(p + S) holds position
// p + S - after + r (a cached row of src when before p, else a new row), rows from
// `after` on are zero (attention.rs:840-862). src is the past cache, or a copy of
// it when present is the same buffer (rows move towards the front).
__global__ __launch_bounds__(256) void gqa_sw_present_kernel(
    const uint32_t* __restrict__ src, const uint32_t* __restrict__ knew, uint32_t* __restrict__ dst,
    const int* __restrict__ seqlens, int S, int KV, int cap, int window, int row_words,
    int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int w = (int)(i % row_words);
        const int64_t rr = i / row_words;
        const int r = (int)(rr % cap);
        const int64_t slab = rr / cap;
        const int b = (int)(slab / KV);
        const int64_t p = max((int64_t)seqlens[b] + 1 - S, (int64_t)0);
        const int gap = cap - window + 1;
        const int64_t after = sw_cache_end(p + S, cap, gap);
        uint32_t x = 0u;
        if (r < after) {
            const int64_t a = p + S - after + r;
            x = a < p ? src[(slab * cap + (a - p + sw_cache_end(p, cap, gap))) * row_words + w]
                      : knew[(slab * S + (a - p)) * row_words + w];
        }
        dst[i] = x;
    }
}

// grid (B*S*H), block 256 = 16 teams of 16 lanes; lane l of a team holds dims
// l, l+16, ..., l+16*(E-1) with E = hd / 16.
template <typename T>
__global__ __launch_bounds__(256) void gqa_ex_attn_kernel(
    const float* __restrict__ qf, const T* __restrict__ pk, const T* __restrict__ pv,
    const T* __restrict__ bias, int64_t bias_sb, int64_t bias_sh, int64_t bias_ss,
    T* __restrict__ out, int S, int H, int KV, int hd, int64_t pcap, int vp, float scale) {
    __shared__ float s_m[kTeams], s_l[kTeams];
    __shared__ float s_acc[kTeams][kMaxHead];
    const int row = blockIdx.x;  // (b*S + s)*H + h
    const int h = row % H;
    const int bs = row / H;
    const int b = bs / S, s = bs % S;
    const int G = H / KV;
    const int kh = h / G;
    const int team = threadIdx.x / kTeamLanes;
    const int lt = threadIdx.x % kTeamLanes;
    const int E = hd / kTeamLanes;
    const int nk = vp + s + 1;  // causal: keys [0, vp + s]
    const float* qrow = qf + (int64_t)row * hd;
    const T* kb = pk + ((int64_t)b * KV + kh) * pcap * hd;
    const T* vb = pv + ((int64_t)b * KV + kh) * pcap * hd;
    const T* brow = bias ? bias + b * bias_sb + h * bias_sh + s * bias_ss : nullptr;

    float qv[kMaxPerLane], acc[kMaxPerLane];
#pragma unroll
    for (int e = 0; e < kMaxPerLane; ++e) {
        qv[e] = e < E ? qrow[lt + kTeamLanes * e] : 0.f;
        acc[e] = 0.f;
    }
    float m = -INFINITY, l = 0.f;
    // Every lane runs the same trip count; a team whose key is past the end skips it.
    for (int base = 0; base < nk; base += kTeams) {
        const int j = base + team;
        const bool valid = j < nk;
        const T* kr = kb + (int64_t)(valid ? j : 0) * hd;
        float dot = 0.f;
#pragma unroll
        for (int e = 0; e < kMaxPerLane; ++e)
            if (e < E) dot += qv[e] * to_f32(kr[lt + kTeamLanes * e]);
        dot = group_sum<kTeamLanes>(dot);
        float sc = dot * scale + (brow && valid ? to_f32(brow[j]) : 0.f);
        if (!valid || sc == -INFINITY) continue;  // uniform over the team's 16 lanes
        const float mn = fmaxf(m, sc);
        const float corr = __expf(m - mn);  // m = -inf -> 0
        const float p = __expf(sc - mn);
        l = l * corr + p;
        const T* vr = vb + (int64_t)j * hd;
#pragma unroll
        for (int e = 0; e < kMaxPerLane; ++e)
            if (e < E) acc[e] = acc[e] * corr + p * to_f32(vr[lt + kTeamLanes * e]);
        m = mn;
    }
    if (lt == 0) {
        s_m[team] = m;
        s_l[team] = l;
    }
#pragma unroll
    for (int e = 0; e < kMaxPerLane; ++e)
        if (e < E) s_acc[team][lt + kTeamLanes * e] = acc[e];
    __syncthreads();
    float M = -INFINITY;
    for (int t = 0; t < kTeams; ++t) M = fmaxf(M, s_m[t]);
    T* orow = out + (int64_t)row * hd;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        float num = 0.f, den = 0.f;
        for (int t = 0; t < kTeams; ++t) {
            if (s_m[t] == -INFINITY) continue;
            const float wt = __expf(s_m[t] - M);
            num += wt * s_acc[t][d];
            den += wt * s_l[t];
        }
        orow[d] = from_f32<T>(num / den);  // every key masked: 0/0, as the softmax gives
    }
}

template <typename T>
int run_gqa_ex(const void* query, const void* key, const void* value, const void* past_key,
               const void* past_value, int64_t cap, int total, const void* cos_c,
               const void* sin_c, int half, int interleaved, const void* qw, const void* kw,
               float eps, const void* bias, int64_t sb, int64_t sh, int64_t ss, void* output,
               void* pk, void* pv, int B, int S, int H, int KV, int hd, float scale, void* ws,
               hipStream_t st) {
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
    const float sc = scale != 0.f ? scale : 1.0f / sqrtf((float)hd);
    const bool aliased = (pk == past_key) && (pv == past_value);
    if (!aliased && cap > 0) {
        // Shared contract into a separate present: all cap rows; growing: the cap past rows.
        const int row_words = hd * (int)sizeof(T) / 4;
        const int64_t total_w = (int64_t)B * KV * cap * row_words;
        const int grid = (int)std::min<int64_t>((total_w + 255) / 256, 65536);
        hipLaunchKernelGGL(kv_rows_copy_kernel, dim3(grid), dim3(256), 0, st,
                           static_cast<const uint32_t*>(past_key), static_cast<uint32_t*>(pk), cap,
                           pcap, cap, row_words, total_w);
        hipLaunchKernelGGL(kv_rows_copy_kernel, dim3(grid), dim3(256), 0, st,
                           static_cast<const uint32_t*>(past_value), static_cast<uint32_t*>(pv),
                           cap, pcap, cap, row_words, total_w);
        if (int rc = check_launch("gqa_ex kv copy")) return rc;
    }
    float* qf = static_cast<float*>(ws);
    hipLaunchKernelGGL((gqa_ex_prep_kernel<T>), dim3(B * S, H + 2 * KV), dim3(64), 0, st, q, k, v,
                       q_stride, kv_stride, static_cast<const T*>(cos_c),
                       static_cast<const T*>(sin_c), half, interleaved, static_cast<const T*>(qw),
                       static_cast<const T*>(kw), eps, qf, static_cast<T*>(pk),
                       static_cast<T*>(pv), S, H, KV, hd, pcap, vp, nullptr, 0);
    if (int rc = check_launch("gqa_ex_prep")) return rc;
    hipLaunchKernelGGL((gqa_ex_attn_kernel<T>), dim3(B * S * H), dim3(256), 0, st, qf,
                       static_cast<const T*>(pk), static_cast<const T*>(pv),
                       static_cast<const T*>(bias), sb, sh, ss, static_cast<T*>(output), S, H, KV,
                       hd, pcap, vp, sc);
    return check_launch("gqa_ex_attn");
}


// Sliding-window cache (attention.rs:725-880): prep (positions from seqlens_k, new
// rows to the workspace), attention over each query's window, then the compacted
// present. When present is the past buffer its rows move towards the front, so
// the past is copied aside first.
template <typename T>
int run_gqa_sliding(const void* query, const void* key, const void* value, const void* past_key,
                    const void* past_value, int cap, const int* seqlens, const void* cos_c,
                    const void* sin_c, int half, int max_pos, int interleaved, const void* qw,
                    const void* kw, float eps, int window, void* output, void* pk, void* pv,
                    int B, int S, int H, int KV, int hd, float scale, void* ws, hipStream_t st) {
    const bool packed = key == nullptr;
    const int64_t q_stride = packed ? (int64_t)(H + 2 * KV) * hd : (int64_t)H * hd;
    const int64_t kv_stride = packed ? q_stride : (int64_t)KV * hd;
    const T* q = static_cast<const T*>(query);
    const T* k = packed ? q + (int64_t)H * hd : static_cast<const T*>(key);
    const T* v = packed ? q + (int64_t)(H + KV) * hd : static_cast<const T*>(value);
    const float sc = scale != 0.f ? scale : 1.0f / sqrtf((float)hd);
    char* w = static_cast<char*>(ws);
    float* qf = reinterpret_cast<float*>(w);
    w += align256((size_t)B * S * H * hd * 4);
    const size_t new_bytes = align256((size_t)B * KV * S * hd * sizeof(T));
    T* knew = reinterpret_cast<T*>(w);
    T* vnew = reinterpret_cast<T*>(w + new_bytes);
    w += 2 * new_bytes;
    hipLaunchKernelGGL((gqa_ex_prep_kernel<T>), dim3(B * S, H + 2 * KV), dim3(64), 0, st, q, k, v,
                       q_stride, kv_stride, static_cast<const T*>(cos_c),
                       static_cast<const T*>(sin_c), half, interleaved, static_cast<const T*>(qw),
                       static_cast<const T*>(kw), eps, qf, knew, vnew, S, H, KV, hd, (int64_t)S, 0,
                       seqlens, max_pos);
    if (int rc = check_launch("gqa_sliding_prep")) return rc;
    hipLaunchKernelGGL((gqa_sw_attn_kernel<T>), dim3(B * S * H), dim3(256), 0, st, qf,
                       static_cast<const T*>(past_key), static_cast<const T*>(past_value), knew,
                       vnew, seqlens, static_cast<T*>(output), S, H, KV, hd, cap, window, sc);
    if (int rc = check_launch("gqa_sliding_attn")) return rc;
    const int row_words = hd * (int)sizeof(T) / 4;
    const int64_t total_w = (int64_t)B * KV * cap * row_words;
    if (total_w == 0) return ORTMI_OK;
    const int grid = (int)std::min<int64_t>((total_w + 255) / 256, 65536);
    const void* srcs[2] = {past_key, past_value};
    const T* news[2] = {knew, vnew};
    void* dsts[2] = {pk, pv};
    for (int i = 0; i < 2; ++i) {
        const uint32_t* src = static_cast<const uint32_t*>(srcs[i]);
        if (srcs[i] == dsts[i]) {  // in place: read the old rows from a copy
            uint32_t* copy = reinterpret_cast<uint32_t*>(w);
            hipLaunchKernelGGL(kv_rows_copy_kernel, dim3(grid), dim3(256), 0, st, src, copy,
                               (int64_t)cap, (int64_t)cap, (int64_t)cap, row_words, total_w);
            src = copy;
        }
        hipLaunchKernelGGL(gqa_sw_present_kernel, dim3(grid), dim3(256), 0, st, src,
                           reinterpret_cast<const uint32_t*>(news[i]),
                           static_cast<uint32_t*>(dsts[i]), seqlens, S, KV, cap, window,
                           row_words, total_w);
        if (int rc = check_launch("gqa_sliding_present")) return rc;
    }
    return ORTMI_OK;
}

}  // namespace
}  // namespace ortmi

using namespace ortmi;

extern "C" size_t ortmi_group_query_attention_ex_workspace_size(int64_t batch, int64_t seq_len,
                                                                int64_t num_heads,
                                                                int64_t head_size) {
    if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || head_size <= 0) return 0;
    return align256((size_t)batch * seq_len * num_heads * head_size * 4);
}

extern "C" int ortmi_group_query_attention_ex(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, int32_t total_sequence_length, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, const void* q_norm_weight,
    const void* k_norm_weight, float qk_norm_epsilon, const void* attention_bias,
    int64_t bias_batch, int64_t bias_heads, int64_t bias_rows, int64_t bias_cols, void* output,
    void* present_key, void* present_value, int64_t batch, int64_t seq_len, int64_t num_heads,
    int64_t kv_num_heads, int64_t head_size, float scale, int32_t rotary_interleaved,
    int32_t dtype, void* workspace, size_t workspace_bytes, void* stream) {
    // Claim/op contract of rust/src/ops/attention.rs:1520-1745 and 556-952.
    ORTMI_REQUIRE(num_heads > 0 && kv_num_heads > 0 && num_heads % kv_num_heads == 0,
                  "GroupQueryAttention: num_heads must be a positive multiple of kv_num_heads");
    ORTMI_REQUIRE(head_size > 0 && head_size % 16 == 0 && head_size <= 256,
                  "GroupQueryAttention: head_size must be a multiple of 16 up to 256");
    ORTMI_REQUIRE(batch > 0 && seq_len > 0 && past_cap >= 0 && num_heads <= 65535 &&
                      batch * seq_len * num_heads <= 0x7fffffffLL,
                  "GroupQueryAttention: bad shape");
    ORTMI_REQUIRE(query && output && present_key && present_value,
                  "GroupQueryAttention: null tensor");
    ORTMI_REQUIRE((key == nullptr) == (value == nullptr),
                  "GroupQueryAttention: key and value must both be given or both be packed");
    ORTMI_REQUIRE(past_cap == 0 || (past_key && past_value), "GroupQueryAttention: null past");
    ORTMI_REQUIRE((q_norm_weight == nullptr) == (k_norm_weight == nullptr),
                  "GroupQueryAttention: q_norm_weight and k_norm_weight must be provided together");
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
    int64_t sb = 0, sh = 0, ss = 0;
    if (attention_bias) {
        ORTMI_REQUIRE((bias_batch == 1 || bias_batch == batch) &&
                          (bias_heads == 1 || bias_heads == num_heads) && bias_rows >= seq_len &&
                          bias_cols >= vp + seq_len,
                      "GroupQueryAttention: attention_bias must be [batch or 1, num_heads or 1, "
                      ">= sequence_length, >= attended keys]");
        ss = bias_cols;
        sh = bias_heads > 1 ? bias_rows * bias_cols : 0;
        sb = bias_batch > 1 ? bias_heads * bias_rows * bias_cols : 0;
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
    const size_t need =
        ortmi_group_query_attention_ex_workspace_size(batch, seq_len, num_heads, head_size);
    if (!workspace || workspace_bytes < need)
        return fail(ORTMI_E_WORKSPACE, "GroupQueryAttention: workspace too small");
    hipStream_t st = as_stream(stream);
#define ORTMI_GQA_EX(T)                                                                          \
    return run_gqa_ex<T>(query, key, value, past_key, past_value, past_cap,                      \
                         total_sequence_length, cos_cache, sin_cache, (int)rotary_half,          \
                         rotary_interleaved, q_norm_weight, k_norm_weight, qk_norm_epsilon,      \
                         attention_bias, sb, sh, ss, output, present_key, present_value,         \
                         (int)batch, (int)seq_len, (int)num_heads, (int)kv_num_heads,            \
                         (int)head_size, scale, workspace, st)
    if (dtype == ORTMI_F32) ORTMI_GQA_EX(float);
    if (dtype == ORTMI_F16) ORTMI_GQA_EX(half_t);
    if (dtype == ORTMI_BF16) ORTMI_GQA_EX(uint16_t);
#undef ORTMI_GQA_EX
    return fail(ORTMI_E_INVALID, "GroupQueryAttention: dtype must be fp32, fp16 or bf16");
}

extern "C" size_t ortmi_group_query_attention_sliding_workspace_size(int64_t batch,
                                                                     int64_t seq_len,
                                                                     int64_t num_heads,
                                                                     int64_t kv_num_heads,
                                                                     int64_t head_size,
                                                                     int64_t past_cap) {
    if (batch <= 0 || seq_len <= 0 || num_heads <= 0 || kv_num_heads <= 0 || head_size <= 0 ||
        past_cap < 0)
        return 0;
    // fp32 queries, new K/V rows and one past copy, sized for 4-byte elements.
    return align256((size_t)batch * seq_len * num_heads * head_size * 4) +
           2 * align256((size_t)batch * kv_num_heads * seq_len * head_size * 4) +
           align256((size_t)batch * kv_num_heads * past_cap * head_size * 4);
}

extern "C" int ortmi_group_query_attention_sliding(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, const int32_t* seqlens_k, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, const void* q_norm_weight,
    const void* k_norm_weight, float qk_norm_epsilon, int64_t local_window_size, void* output,
    void* present_key, void* present_value, int64_t batch, int64_t seq_len, int64_t num_heads,
    int64_t kv_num_heads, int64_t head_size, float scale, int32_t rotary_interleaved,
    int32_t dtype, void* workspace, size_t workspace_bytes, void* stream) {
    // attention.rs:725-735 and the claim at 1552-1575.
    ORTMI_REQUIRE(num_heads > 0 && kv_num_heads > 0 && num_heads % kv_num_heads == 0,
                  "GroupQueryAttention: num_heads must be a positive multiple of kv_num_heads");
    ORTMI_REQUIRE(head_size > 0 && head_size % 16 == 0 && head_size <= 256,
                  "GroupQueryAttention: head_size must be a multiple of 16 up to 256");
    ORTMI_REQUIRE(batch > 0 && seq_len > 0 && num_heads <= 65535 && past_cap <= 0x7fffffffLL &&
                      batch * seq_len * num_heads <= 0x7fffffffLL,
                  "GroupQueryAttention: bad shape");
    ORTMI_REQUIRE(local_window_size > 0 && local_window_size <= past_cap,
                  "GroupQueryAttention: sliding cache requires 0 < local_window_size <= capacity");
    ORTMI_REQUIRE(query && output && present_key && present_value && past_key && past_value &&
                      seqlens_k,
                  "GroupQueryAttention: null tensor");
    ORTMI_REQUIRE((key == nullptr) == (value == nullptr),
                  "GroupQueryAttention: key and value must both be given or both be packed");
    ORTMI_REQUIRE((q_norm_weight == nullptr) == (k_norm_weight == nullptr),
                  "GroupQueryAttention: q_norm_weight and k_norm_weight must be provided together");
    const bool rotary = cos_cache != nullptr;
    ORTMI_REQUIRE(rotary == (sin_cache != nullptr),
                  "GroupQueryAttention: cos_cache and sin_cache must both be given");
    if (rotary)
        ORTMI_REQUIRE(rotary_half > 0 && 2 * rotary_half <= head_size && max_pos > 0,
                      "GroupQueryAttention: rotary dim exceeds head_size");
    if ((past_key == present_key) != (past_value == present_value))
        return fail(ORTMI_E_INVALID, "GroupQueryAttention: present_key/value alias mismatch");
    const size_t need = ortmi_group_query_attention_sliding_workspace_size(
        batch, seq_len, num_heads, kv_num_heads, head_size, past_cap);
    if (!workspace || workspace_bytes < need)
        return fail(ORTMI_E_WORKSPACE, "GroupQueryAttention: workspace too small");
    hipStream_t st = as_stream(stream);
#define ORTMI_GQA_SW(T)                                                                          \
    return run_gqa_sliding<T>(query, key, value, past_key, past_value, (int)past_cap, seqlens_k,  \
                              cos_cache, sin_cache, (int)rotary_half, (int)max_pos,              \
                              rotary_interleaved, q_norm_weight, k_norm_weight, qk_norm_epsilon, \
                              (int)local_window_size, output, present_key, present_value,        \
                              (int)batch, (int)seq_len, (int)num_heads, (int)kv_num_heads,       \
                              (int)head_size, scale, workspace, st)
    if (dtype == ORTMI_F32) ORTMI_GQA_SW(float);
    if (dtype == ORTMI_F16) ORTMI_GQA_SW(half_t);
    if (dtype == ORTMI_BF16) ORTMI_GQA_SW(uint16_t);
#undef ORTMI_GQA_SW
    return fail(ORTMI_E_INVALID, "GroupQueryAttention: dtype must be fp32, fp16 or bf16");
}
