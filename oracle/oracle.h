/*
 * oracle.h - CPU restatement of the reference's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls
 * this code; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * use it, and only as the checker (or as the timed CPU baseline).
 *
 * Every entry point cites the reference file:line whose semantics it restates
 * (paths relative to the reference repository root). Arithmetic is carried out in
 * fp64 wherever the reference's contract is "fp32 or better", so the oracle is a
 * tighter target than either ORT's CPU EP or MLX. Where the reference
 * materialises an intermediate in the op dtype (fp16 rotary outputs, fp16
 * residual sums, fp16 KV-cache writes), the `round16` flag reproduces that
 * rounding with round-to-nearest-even.
 */
#ifndef ORT_MI355X_ORACLE_H
#define ORT_MI355X_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE binary16 <-> binary32, round-to-nearest-even. */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_f16_to_f32_n(const uint16_t* src, float* dst, int64_t n);
void orc_f32_to_f16_n(const float* src, uint16_t* dst, int64_t n);

/*
 * MatMulNBits dequantisation, W[n*K + k] = (q(n,k) - zp(n,k/bs)) * s(n,k/bs).
 * Layout per rust/src/ops/quant.rs:679-697 (repack loop: byte
 * ((n*nb + blk)*bs*bits/8 + within*bits/8), low nibble first) and
 * quant.rs:906-919 (packed 4-bit zero points: byte n*ceil(nb/2) + b/2, low nibble
 * for even b). Absent zero points default to 2^(bits-1) (quant.rs:824-861).
 * Returns 0, or -1 on an unsupported bits value.
 */
int orc_mnb_dequant(const uint8_t* B, const float* scales, const uint8_t* zp,
                    int64_t N, int64_t K, int bits, int block, float* W);

/*
 * MatMulNBits, Y[M,N] = A[M,K] . W^T with W as above, fp64 accumulation
 * (rust/src/ops/quant.rs:986-1130; K is zero-padded to nb*bs at quant.rs:1034-1039,
 * which contributes nothing). nthreads <= 0 uses all OpenMP threads.
 */
int orc_mnb_matmul(const float* A, const uint8_t* B, const float* scales, const uint8_t* zp,
                   int64_t M, int64_t N, int64_t K, int bits, int block, double* Y,
                   int nthreads);

/*
 * fast.c: the CPU baseline's form of the same product for 4-bit weights, fp32
 * accumulation with AVX2/FMA (scales fp32, or fp16 bits when scale_f16; blocks of
 * 32, 64, 96 or 128 codes, K a multiple of the block). -1 when the form or the CPU is outside
 * it. Pinned against orc_mnb_matmul by tests/test_oracle.py.
 */
int orc_mnb_matmul_fast(const float* A, int64_t M, const uint8_t* B, const void* scales,
                        int scale_f16, const uint8_t* zp, int64_t N, int64_t K, int block,
                        float* Y, int nthreads);

/*
 * Rotary embedding over a strided tensor: element (b, s, n, d) lives at
 * x[b*sb + s*ss + n*sn + d]. Token (b, s) uses cache row rows[b*S + s].
 * Rotates dims [offset, offset + 2*half) of each head; other dims pass through.
 * Non-interleaved (rotate-half) and interleaved forms per
 * rust/src/ops/attention.rs:1234-1282 (rope_apply) and attention.rs:417-461.
 */
void orc_rotary(const float* x, float* y, int B, int S, int NH, int hd,
                int64_t sb, int64_t ss, int64_t sn, const int64_t* rows,
                const float* cos_c, const float* sin_c, int half, int interleaved,
                int offset, int round16);

/*
 * GroupQueryAttention per rust/src/ops/attention.rs:556-952:
 *  - valid_past = total_seq_len - S (uniform over the batch; seqlens_k is not
 *    consulted outside sliding mode, attention.rs:642-651);
 *  - shared-buffer contract iff cap > valid_past (present = past buffer with the S
 *    new rows written at valid_past), otherwise growing (present = concat(past,
 *    new), cap + S rows); a valid_past outside [0, cap] falls back to growing;
 *  - RoPE on Q and K at positions valid_past .. valid_past+S-1;
 *  - causal top-left SDPA: query i attends keys j <= valid_past + i
 *    (attention.rs:171-189, 264-285).
 * q: [B,S,H*hd]; if k == NULL, q is packed [B,S,(H+2KV)*hd] (attention.rs:564-596).
 * past_k/past_v: [B,KV,cap,hd]. present_*: [B,KV,pcap,hd] with pcap returned by
 * orc_gqa_contract. out: [B,S,H*hd] (fp64-accurate, not rounded).
 * Returns the contract (0 growing, 1 shared) or -1 on bad arguments.
 */
int orc_gqa_contract(int total_seq_len, int S, int64_t cap, int* valid_past, int64_t* pcap);
int orc_gqa(const float* q, const float* k, const float* v,
            const float* past_k, const float* past_v, int64_t cap, int total_seq_len,
            const float* cos_c, const float* sin_c, int half, int interleaved,
            int B, int S, int H, int KV, int hd, float scale, int round16,
            float* out, float* present_k, float* present_v);
/*
 * orc_gqa plus the optional GroupQueryAttention inputs the reference accepts
 * (rust/src/ops/attention.rs:1520-1720):
 *  - q_norm_w/k_norm_w [hd] (inputs 14/15): per-head RMS norm with qk_eps applied to
 *    q and to the new k before RoPE (attention.rs:663-670);
 *  - bias (input 10): additive scores mask; the row for (batch b, head h, query s)
 *    starts at bias + b*bias_sb + h*bias_sh + s*bias_ss and is indexed by key
 *    position; it is added to scale*q.k and the causal mask still applies
 *    (attention.rs:256-285). Broadcast dimensions carry stride 0.
 * round16 = 2 rounds to bf16 where 1 rounds to fp16.
 */
int orc_gqa_ex(const float* q, const float* k, const float* v, const float* past_k,
               const float* past_v, int64_t cap, int total_seq_len, const float* cos_c,
               const float* sin_c, int half, int interleaved, int B, int S, int H, int KV, int hd,
               float scale, int round16, const float* q_norm_w, const float* k_norm_w,
               float qk_eps, const float* bias, int64_t bias_sb, int64_t bias_sh,
               int64_t bias_ss, float* out, float* present_k, float* present_v);

/*
 * PagedAttention per rust/src/ops/attention.rs:2495-2744, with RoPE read straight
 * from the cos/sin cache rows as in the reference's test oracle
 * tests/ops/test_paged_attention.py:29-143 (_paged_ref):
 *  - per sequence b, tokens cum[b]..cum[b+1], past = past_lens[b];
 *  - optional QK RMS-norm (attention.rs:2612-2616) then RoPE at positions
 *    past+j on dims [rot_offset, rot_offset+2*half) (attention.rs:2619-2623);
 *  - new K/V written to slot slot_mapping[t] (skipped when < 0) or
 *    bt[b, p/blk]*blk + p%blk (attention.rs:2630-2673);
 *  - keys p < past read from the (updated) cache, p >= past from the new rows;
 *  - causal fp32 SDPA with optional per-head sink logit (attention.rs:2423-2452).
 * LATENT layout (v == NULL, vcache == NULL): values are the first vhd dims of the
 * keys (attention.rs:2500-2505, 2624-2628).
 * kcache/vcache are updated in place. out: [T, H*vhd].
 */
int orc_paged_attention(const float* q, const float* k, const float* v,
                        float* kcache, float* vcache, int64_t nblk, int blk,
                        const int32_t* cum, const int32_t* past_lens, const int32_t* bt,
                        int batch, int maxb,
                        const float* cos_c, const float* sin_c, int half, int interleaved,
                        int rot_offset, const int32_t* slot_mapping, const float* head_sink,
                        const float* q_norm_w, const float* k_norm_w, float qk_eps,
                        int H, int KV, int hd, int vhd, float scale, int round16, float* out);

/*
 * SimplifiedLayerNormalization / SkipSimplifiedLayerNormalization per
 * rust/src/ops/norm.rs:175-185 and norm.rs:231-248:
 *   r = x (+ skip) (+ bias), rounded to fp16 when round16 (the reference adds in
 *   the op dtype before normalising); y = r / sqrt(mean(r^2) + eps) * gamma.
 * skip/bias/residual may be NULL.
 */
void orc_rms_norm(const float* x, const float* skip, const float* bias, const float* gamma,
                  int64_t rows, int64_t D, float eps, int round16, float* y, float* residual);

#ifdef __cplusplus
}
#endif
#endif
