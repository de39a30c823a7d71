/*
 * oracle.c - CPU restatement of the reference's hot-path arithmetic.
 * TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the shipped library.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 --- */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    float f;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in binary32 */
        f = (float)man * 5.9604644775390625e-08f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14 */
        float v;
        memcpy(&v, &ax, 4);
        float r = v * 16777216.0f; /* exact power-of-two scaling, r < 1024 */
        uint32_t i = (uint32_t)r;
        float frac = r - (float)i;
        if (frac > 0.5f || (frac == 0.5f && (i & 1u))) i++;
        return (uint16_t)(sign | i);
    }
    uint32_t mant = ax & 0x7fffffu;
    uint32_t e = (ax >> 23) - 112u;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry into exponent is correct */
    return (uint16_t)(sign | h);
}

void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f16_to_f32(src[i]);
}

void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_f16(src[i]);
}

/* Round-to-nearest-even to bfloat16 (the top 16 bits of the binary32 pattern). */
static inline float rbf16(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return v;
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    memcpy(&v, &u, 4);
    return v;
}

/* round16: 0 keeps fp32, 1 rounds to fp16, 2 rounds to bf16. */
static inline float r16(float v, int round16) {
    if (round16 == 2) return rbf16(v);
    return round16 ? orc_f16_to_f32(orc_f32_to_f16(v)) : v;
}

/* --------------------------------------------------------- MatMulNBits --- */

/* Quantised code of element (n, k): rust/src/ops/quant.rs:679-697. */
static inline int mnb_code(const uint8_t* B, int64_t nb, int64_t n, int64_t k, int bits,
                           int block) {
    int64_t blk = k / block, within = k % block;
    int64_t blob = (int64_t)block * bits / 8;
    if (bits == 4) {
        uint8_t byte = B[(n * nb + blk) * blob + within / 2];
        return (within & 1) ? (byte >> 4) : (byte & 0x0f);
    }
    return B[(n * nb + blk) * blob + within];
}

/* Zero point of block (n, b): rust/src/ops/quant.rs:906-919 (4-bit), 8-bit is one
 * byte per block; absent -> 2^(bits-1) (quant.rs:824-861 symmetric bias). */
static inline int mnb_zp(const uint8_t* zp, int64_t nb, int64_t n, int64_t b, int bits) {
    if (!zp) return 1 << (bits - 1);
    if (bits == 4) {
        int64_t cols = (nb + 1) / 2;
        uint8_t byte = zp[n * cols + b / 2];
        return (b & 1) ? (byte >> 4) : (byte & 0x0f);
    }
    return zp[n * nb + b];
}

int orc_mnb_dequant(const uint8_t* B, const float* scales, const uint8_t* zp, int64_t N,
                    int64_t K, int bits, int block, float* W) {
    if (bits != 4 && bits != 8) return -1;
    if (block <= 0 || (block * bits) % 8) return -1;
    int64_t nb = (K + block - 1) / block;
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            int64_t b = k / block;
            int q = mnb_code(B, nb, n, k, bits, block);
            int z = mnb_zp(zp, nb, n, b, bits);
            W[n * K + k] = (float)(q - z) * scales[n * nb + b];
        }
    return 0;
}

int orc_mnb_matmul(const float* A, const uint8_t* B, const float* scales, const uint8_t* zp,
                   int64_t M, int64_t N, int64_t K, int bits, int block, double* Y,
                   int nthreads) {
    if (bits != 4 && bits != 8) return -1;
    if (block <= 0 || (block * bits) % 8) return -1;
    int64_t nb = (K + block - 1) / block;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel
    {
        double* w = (double*)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1));
#pragma omp for schedule(static)
        for (int64_t n = 0; n < N; ++n) {
            for (int64_t k = 0; k < K; ++k) {
                int64_t b = k / block;
                int q = mnb_code(B, nb, n, k, bits, block);
                int z = mnb_zp(zp, nb, n, b, bits);
                w[k] = (double)(q - z) * (double)scales[n * nb + b];
            }
            for (int64_t m = 0; m < M; ++m) {
                const float* a = A + m * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += (double)a[k] * w[k];
                Y[m * N + n] = acc;
            }
        }
        free(w);
    }
    return 0;
}

/* -------------------------------------------------------------- RoPE --- */

/* Rotate one head vector in place-free fashion: x -> y over dims
 * [offset, offset+2*half). attention.rs:1261-1279 (rotate-half: o1 = x1*c - x2*s,
 * o2 = x1*s + x2*c) and attention.rs:1263-1276 interleaved pairs (2i, 2i+1). */
static void rope_vec(const float* x, float* y, int hd, const float* c, const float* s,
                     int half, int interleaved, int offset, int round16) {
    for (int d = 0; d < hd; ++d) y[d] = x[d];
    const float* xr = x + offset;
    float* yr = y + offset;
    for (int i = 0; i < half; ++i) {
        double ci = c[i], si = s[i];
        double a, b;
        int ia, ib;
        if (interleaved) {
            ia = 2 * i;
            ib = 2 * i + 1;
        } else {
            ia = i;
            ib = i + half;
        }
        a = xr[ia];
        b = xr[ib];
        yr[ia] = r16((float)(a * ci - b * si), round16);
        yr[ib] = r16((float)(b * ci + a * si), round16);
    }
}

void orc_rotary(const float* x, float* y, int B, int S, int NH, int hd, int64_t sb,
                int64_t ss, int64_t sn, const int64_t* rows, const float* cos_c,
                const float* sin_c, int half, int interleaved, int offset, int round16) {
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < S; ++s) {
            int64_t row = rows[(int64_t)b * S + s];
            const float* c = cos_c + row * half;
            const float* sn_ = sin_c + row * half;
            for (int n = 0; n < NH; ++n) {
                int64_t base = b * sb + s * ss + n * sn;
                rope_vec(x + base, y + base, hd, c, sn_, half, interleaved, offset, round16);
            }
        }
}

/* ------------------------------------------------------ attention core --- */

/* One query row against `nk` keys (rows of kbuf with stride kstride), values
 * likewise; keys j > last are masked (causal). Optional sink logit joins only the
 * denominator (attention.rs:2423-2452; test_paged_attention.py:130-134). */
static void attend_row(const float* qv, int hd, const float* const* krows,
                       const float* const* vrows, int nk, int vhd, int last, double scale,
                       const float* sink, const float* bias, double* scores, float* out) {
    double mx = -INFINITY;
    for (int j = 0; j < nk; ++j) {
        if (j > last) {
            scores[j] = -INFINITY;
            continue;
        }
        double acc = 0.0;
        for (int d = 0; d < hd; ++d) acc += (double)qv[d] * (double)krows[j][d];
        scores[j] = acc * scale + (bias ? (double)bias[j] : 0.0);
        if (scores[j] > mx) mx = scores[j];
    }
    if (sink && (double)*sink > mx) mx = *sink;
    double denom = 0.0;
    for (int j = 0; j < nk; ++j) {
        scores[j] = (j > last || scores[j] == -INFINITY) ? 0.0 : exp(scores[j] - mx);
        denom += scores[j];
    }
    if (sink) denom += exp((double)*sink - mx);
    /* Each out[d] sums scores[j] * v[j][d] over j in ascending order (keys past
     * `last` carry weight 0 and are skipped); j runs in the outer loop so the V
     * rows are read contiguously. */
    double acc[512];
    for (int d = 0; d < vhd; ++d) acc[d] = 0.0;
    const int nj = last + 1 < nk ? last + 1 : nk;
    for (int j = 0; j < nj; ++j) {
        const double w = scores[j];
        const float* vr = vrows[j];
        for (int d = 0; d < vhd; ++d) acc[d] += w * (double)vr[d];
    }
    for (int d = 0; d < vhd; ++d) out[d] = (float)(acc[d] / denom);
}

/* ---------------------------------------------------------------- GQA --- */

/* RMS-normalise one head vector with per-dimension weights (QK-norm). */
static void rms_vec(const float* x, float* y, int d, const float* w, float eps, int round16) {
    double ss = 0.0;
    for (int i = 0; i < d; ++i) ss += (double)x[i] * (double)x[i];
    double inv = 1.0 / sqrt(ss / d + (double)eps);
    for (int i = 0; i < d; ++i) y[i] = r16((float)((double)x[i] * inv * (double)w[i]), round16);
}


int orc_gqa_contract(int total_seq_len, int S, int64_t cap, int* valid_past, int64_t* pcap) {
    /* attention.rs:636-651 */
    int vp = total_seq_len - S;
    int shared;
    if (vp < 0 || vp > cap) {
        shared = 0;
        vp = (int)cap;
    } else {
        shared = cap > vp;
    }
    if (valid_past) *valid_past = vp;
    if (pcap) *pcap = shared ? cap : cap + S;
    return shared;
}

int orc_gqa_ex(const float* q, const float* k, const float* v, const float* past_k,
               const float* past_v, int64_t cap, int total_seq_len, const float* cos_c,
               const float* sin_c, int half, int interleaved, int B, int S, int H, int KV, int hd,
               float scale, int round16, const float* q_norm_w, const float* k_norm_w,
               float qk_eps, const float* bias, int64_t bias_sb, int64_t bias_sh,
               int64_t bias_ss, float* out, float* present_k, float* present_v) {
    if (H <= 0 || KV <= 0 || H % KV || hd <= 0 || hd > 512 || S <= 0) return -1;
    if (cos_c && 2 * half > hd) return -1;
    int vp;
    int64_t pcap;
    int shared = orc_gqa_contract(total_seq_len, S, cap, &vp, &pcap);
    if (shared && (int64_t)vp + S > cap) return -1; /* new rows would not fit the buffer */
    int g = H / KV;
    double sc = scale != 0.0f ? (double)scale : 1.0 / sqrt((double)hd);
    int packed = (k == NULL);
    int64_t qrow = packed ? (int64_t)(H + 2 * KV) * hd : (int64_t)H * hd;
    int64_t krow = packed ? qrow : (int64_t)KV * hd;
    const float* kbase = packed ? q + (int64_t)H * hd : k;
    const float* vbase = packed ? q + (int64_t)(H + KV) * hd : v;

    float* qr = (float*)malloc(sizeof(float) * (size_t)hd);
    float* kr = (float*)malloc(sizeof(float) * (size_t)hd);

    /* present = past (growing: rows [0,cap); shared: the whole buffer). */
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < KV; ++h)
            for (int64_t t = 0; t < cap; ++t) {
                const float* srck = past_k + (((int64_t)b * KV + h) * cap + t) * hd;
                const float* srcv = past_v + (((int64_t)b * KV + h) * cap + t) * hd;
                float* dk = present_k + (((int64_t)b * KV + h) * pcap + t) * hd;
                float* dv = present_v + (((int64_t)b * KV + h) * pcap + t) * hd;
                memcpy(dk, srck, sizeof(float) * (size_t)hd);
                memcpy(dv, srcv, sizeof(float) * (size_t)hd);
            }
    /* New K (rotated) and V at rows vp..vp+S-1 (attention.rs:893-908). */
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < S; ++s) {
            const float* krow_p = kbase + ((int64_t)b * S + s) * krow;
            const float* vrow_p = vbase + ((int64_t)b * S + s) * krow;
            for (int h = 0; h < KV; ++h) {
                const float* kin = krow_p + (int64_t)h * hd;
                /* QK-norm, then RoPE (attention.rs:663-708). */
                if (k_norm_w) {
                    rms_vec(kin, qr, hd, k_norm_w, qk_eps, round16);
                    kin = qr;
                }
                if (cos_c) {
                    int64_t pos = vp + s;
                    rope_vec(kin, kr, hd, cos_c + pos * half, sin_c + pos * half, half,
                             interleaved, 0, round16);
                } else {
                    for (int d = 0; d < hd; ++d) kr[d] = kin[d];
                }
                float* dk = present_k + (((int64_t)b * KV + h) * pcap + vp + s) * hd;
                float* dv = present_v + (((int64_t)b * KV + h) * pcap + vp + s) * hd;
                memcpy(dk, kr, sizeof(float) * (size_t)hd);
                memcpy(dv, vrow_p + (int64_t)h * hd, sizeof(float) * (size_t)hd);
            }
        }
    /* Attention over [0, vp+S) with the query at absolute position vp+s. Rows
     * (b, s, h) are independent and run in parallel; each row's arithmetic does
     * not depend on the thread count. */
    int nk = vp + S;
    const int64_t nrows = (int64_t)B * S * H;
#pragma omp parallel
    {
        float* qrt = (float*)malloc(sizeof(float) * (size_t)hd);
        float* qnt = (float*)malloc(sizeof(float) * (size_t)hd);
        double* sbuf = (double*)malloc(sizeof(double) * (size_t)(pcap + 1));
        const float** kpt = (const float**)malloc(sizeof(float*) * (size_t)(pcap + 1));
        const float** vpt = (const float**)malloc(sizeof(float*) * (size_t)(pcap + 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t row = 0; row < nrows; ++row) {
            const int h = (int)(row % H);
            const int s = (int)((row / H) % S);
            const int b = (int)(row / ((int64_t)H * S));
            const float* qin = q + ((int64_t)b * S + s) * qrow + (int64_t)h * hd;
            if (q_norm_w) {
                rms_vec(qin, qnt, hd, q_norm_w, qk_eps, round16);
                qin = qnt;
            }
            if (cos_c) {
                int64_t pos = vp + s;
                rope_vec(qin, qrt, hd, cos_c + pos * half, sin_c + pos * half, half,
                         interleaved, 0, round16);
            } else {
                for (int d = 0; d < hd; ++d) qrt[d] = qin[d];
            }
            int kvh = h / g;
            for (int j = 0; j < nk; ++j) {
                kpt[j] = present_k + (((int64_t)b * KV + kvh) * pcap + j) * hd;
                vpt[j] = present_v + (((int64_t)b * KV + kvh) * pcap + j) * hd;
            }
            float* o = out + ((int64_t)b * S + s) * (int64_t)H * hd + (int64_t)h * hd;
            /* attention_bias (input 10): an additive mask row over the key
             * positions (attention.rs:1593-1640), broadcast over batch/heads. */
            const float* brow = bias ? bias + b * bias_sb + h * bias_sh + s * bias_ss : NULL;
            attend_row(qrt, hd, kpt, vpt, nk, hd, vp + s, sc, NULL, brow, sbuf, o);
        }
        free(qrt);
        free(qnt);
        free(sbuf);
        free(kpt);
        free(vpt);
    }
    free(qr);
    free(kr);
    (void)shared;
    return shared;
}

int orc_gqa(const float* q, const float* k, const float* v, const float* past_k,
            const float* past_v, int64_t cap, int total_seq_len, const float* cos_c,
            const float* sin_c, int half, int interleaved, int B, int S, int H, int KV, int hd,
            float scale, int round16, float* out, float* present_k, float* present_v) {
    return orc_gqa_ex(q, k, v, past_k, past_v, cap, total_seq_len, cos_c, sin_c, half,
                      interleaved, B, S, H, KV, hd, scale, round16, NULL, NULL, 0.f, NULL, 0, 0, 0,
                      out, present_k, present_v);
}

/* ------------------------------------------------------ PagedAttention --- */


int orc_paged_attention(const float* q, const float* k, const float* v, float* kcache,
                        float* vcache, int64_t nblk, int blk, const int32_t* cum,
                        const int32_t* past_lens, const int32_t* bt, int batch, int maxb,
                        const float* cos_c, const float* sin_c, int half, int interleaved,
                        int rot_offset, const int32_t* slot_mapping, const float* head_sink,
                        const float* q_norm_w, const float* k_norm_w, float qk_eps, int H,
                        int KV, int hd, int vhd, float scale, int round16, float* out) {
    if (H <= 0 || KV <= 0 || H % KV || blk <= 0 || hd > 512 || vhd > 512) return -1;
    int latent = (v == NULL);
    if (latent && vhd > hd) return -1;
    int g = H / KV;
    double sc = scale != 0.0f ? (double)scale : 1.0 / sqrt((double)hd);
    int64_t kslot = (int64_t)KV * hd, vslot = (int64_t)KV * vhd;
    int64_t T = cum[batch];
    float* qn = (float*)malloc(sizeof(float) * (size_t)(T * H * hd + 1));
    float* kn = (float*)malloc(sizeof(float) * (size_t)(T * KV * hd + 1));
    float* tmp = (float*)malloc(sizeof(float) * (size_t)hd);

    for (int b = 0; b < batch; ++b) {
        int s0 = cum[b], s1 = cum[b + 1], nq = s1 - s0;
        if (nq <= 0) continue;
        int pastb = past_lens[b];
        /* QK-norm, then RoPE (attention.rs:2606-2623). */
        for (int i = 0; i < nq; ++i) {
            int64_t t = s0 + i;
            int64_t pos = (int64_t)pastb + i;
            for (int h = 0; h < H; ++h) {
                const float* src = q + t * (int64_t)H * hd + (int64_t)h * hd;
                float* dst = qn + t * (int64_t)H * hd + (int64_t)h * hd;
                if (q_norm_w) rms_vec(src, tmp, hd, q_norm_w, qk_eps, round16);
                else memcpy(tmp, src, sizeof(float) * (size_t)hd);
                if (cos_c)
                    rope_vec(tmp, dst, hd, cos_c + pos * half, sin_c + pos * half, half,
                             interleaved, rot_offset, round16);
                else memcpy(dst, tmp, sizeof(float) * (size_t)hd);
            }
            for (int h = 0; h < KV; ++h) {
                const float* src = k + t * kslot + (int64_t)h * hd;
                float* dst = kn + t * kslot + (int64_t)h * hd;
                if (k_norm_w) rms_vec(src, tmp, hd, k_norm_w, qk_eps, round16);
                else memcpy(tmp, src, sizeof(float) * (size_t)hd);
                if (cos_c)
                    rope_vec(tmp, dst, hd, cos_c + pos * half, sin_c + pos * half, half,
                             interleaved, rot_offset, round16);
                else memcpy(dst, tmp, sizeof(float) * (size_t)hd);
            }
        }
        /* Cache write (attention.rs:2630-2673). */
        for (int i = 0; i < nq; ++i) {
            int64_t t = s0 + i;
            int64_t slot;
            if (slot_mapping) {
                slot = slot_mapping[t];
            } else {
                int64_t p = (int64_t)pastb + i;
                slot = (int64_t)bt[(int64_t)b * maxb + p / blk] * blk + p % blk;
            }
            if (slot < 0 || slot >= nblk * blk) continue;
            for (int h = 0; h < KV; ++h) {
                float* dk = kcache + slot * kslot + (int64_t)h * hd;
                const float* sk = kn + t * kslot + (int64_t)h * hd;
                for (int d = 0; d < hd; ++d) dk[d] = r16(sk[d], round16);
                if (!latent) {
                    float* dv = vcache + slot * vslot + (int64_t)h * vhd;
                    const float* sv = v + t * vslot + (int64_t)h * vhd;
                    for (int d = 0; d < vhd; ++d) dv[d] = r16(sv[d], round16);
                }
            }
        }
        /* Attention: keys [0, past) from the cache, [past, past+nq) new. Rows
         * (head, query) are independent, so they run in parallel; each row's
         * arithmetic does not depend on the thread count. */
        int total = pastb + nq;
        const float** kpa = (const float**)malloc(sizeof(float*) * (size_t)KV * (total + 1));
        const float** vpa = (const float**)malloc(sizeof(float*) * (size_t)KV * (total + 1));
        for (int kvh = 0; kvh < KV; ++kvh) {
            const float** kr = kpa + (int64_t)kvh * total;
            const float** vr = vpa + (int64_t)kvh * total;
            for (int j = 0; j < total; ++j) {
                if (j < pastb) {
                    int64_t slot = (int64_t)bt[(int64_t)b * maxb + j / blk] * blk + j % blk;
                    kr[j] = kcache + slot * kslot + (int64_t)kvh * hd;
                    vr[j] = latent ? kr[j] : vcache + slot * vslot + (int64_t)kvh * vhd;
                } else {
                    int64_t t = s0 + (j - pastb);
                    kr[j] = kn + t * kslot + (int64_t)kvh * hd;
                    vr[j] = latent ? kr[j] : v + t * vslot + (int64_t)kvh * vhd;
                }
            }
        }
#pragma omp parallel
        {
            double* sbuf = (double*)malloc(sizeof(double) * (size_t)(total + 1));
#pragma omp for collapse(2) schedule(dynamic, 8)
            for (int h = 0; h < H; ++h)
                for (int i = 0; i < nq; ++i) {
                    int kvh = h / g;
                    int64_t t = s0 + i;
                    const float* qv = qn + t * (int64_t)H * hd + (int64_t)h * hd;
                    float* o = out + t * (int64_t)H * vhd + (int64_t)h * vhd;
                    attend_row(qv, hd, kpa + (int64_t)kvh * total, vpa + (int64_t)kvh * total,
                               total, vhd, pastb + i, sc, head_sink ? head_sink + h : NULL, NULL,
                               sbuf, o);
                }
            free(sbuf);
        }
        free(kpa);
        free(vpa);
    }
    free(qn);
    free(kn);
    free(tmp);
    return 0;
}

/* ----------------------------------------------------------- RMS norm --- */

void orc_rms_norm(const float* x, const float* skip, const float* bias, const float* gamma,
                  int64_t rows, int64_t D, float eps, int round16, float* y, float* residual) {
    float* r = (float*)malloc(sizeof(float) * (size_t)D);
    for (int64_t i = 0; i < rows; ++i) {
        const float* xi = x + i * D;
        double ss = 0.0;
        for (int64_t d = 0; d < D; ++d) {
            /* The residual sum in fp32, left to right (input + skip, then + bias), as
             * ORT's CPU SkipLayerNorm kernels form input_skip_bias_sum; the sum of
             * two values is one correctly rounded fp32 add either way. */
            float t = xi[d];
            if (skip) t = (float)((double)t + (double)skip[i * D + d]);
            if (bias) t = (float)((double)t + (double)bias[d]);
            r[d] = r16(t, round16 && (skip || bias));
            ss += (double)r[d] * (double)r[d];
        }
        double inv = 1.0 / sqrt(ss / (double)D + (double)eps);
        for (int64_t d = 0; d < D; ++d) {
            y[i * D + d] = (float)((double)r[d] * inv * (double)gamma[d]);
            if (residual) residual[i * D + d] = r[d];
        }
    }
    free(r);
}
