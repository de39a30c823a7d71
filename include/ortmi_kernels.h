/*
 * ortmi_kernels.h - C ABI of the MI355X (gfx950) kernel library
 * (libortmi_kernels.so).
 *
 * This library is the compute backend of the MI355X execution provider. It takes
 * the place that mlx-c / MLX hold in the reference EP: the reference's op
 * translators (rust/src/ops/quant.rs, rust/src/ops/attention.rs,
 * rust/src/ops/norm.rs) bind mlx-c functions through bindgen
 * (rust/build.rs:76-87) and hand them MLX arrays; the MI355X EP's op layer calls
 * these entry points instead, with plain device pointers and sizes.
 *
 * Conventions (all entry points):
 *  - Tensor pointers are device pointers (hipMalloc'd or from the EP's
 *    allocator); scalar sizes are host values; `stream` is a hipStream_t (NULL =
 *    the null stream). Work is enqueued asynchronously on `stream`.
 *  - `dtype` is the ONNX TensorProto element type of the float tensors:
 *    ORTMI_F32 (1), ORTMI_F16 (10) or ORTMI_BF16 (16).
 *  - Return 0 on success, otherwise an ORTMI_E_* code; ortmi_last_error()
 *    returns the calling thread's last message. Errors are detected on the host
 *    before any launch, so a failed call enqueues nothing.
 *  - Workspace, where an entry point needs one, is caller-owned device memory;
 *    the matching *_workspace_size() gives its size. The library itself never
 *    allocates device memory.
 */
#ifndef ORTMI_KERNELS_H
#define ORTMI_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ORTMI_F32 = 1,
    ORTMI_F16 = 10,
    ORTMI_BF16 = 16,
};

enum {
    ORTMI_OK = 0,
    ORTMI_E_INVALID = 1,     /* bad argument / unsupported form */
    ORTMI_E_HIP = 2,         /* HIP runtime error */
    ORTMI_E_WORKSPACE = 3,   /* workspace too small */
};

#define ORTMI_ABI_VERSION 2

int ortmi_abi_version(void);
const char* ortmi_last_error(void);

/*
 * Host-to-device copies of up to ORTMI_SMALL_COPIES small host buffers (at most
 * ORTMI_SMALL_COPY_BYTES bytes in all) in one kernel launch on `stream`: the
 * bytes travel in the launch's arguments, so the host buffers may be pageable and
 * may be reused as soon as the call returns; dst[i] are device pointers that
 * receive bytes[i] bytes each, in stream order. Used by the execution provider's
 * OrtDataTransferImpl::CopyTensors for the per-run feeds of a decode step (input
 * ids and the two length scalars), which as separate DMA copies cost about 6 us
 * each. No counterpart in the reference, whose factory creates no data transfer
 * (rust/src/factory.rs:238-242: MLX memory is unified with the host).
 */
#define ORTMI_SMALL_COPIES 16
#define ORTMI_SMALL_COPY_BYTES 1024
int ortmi_copy_small_h2d(int n, void* const* dst, const void* const* src, const size_t* bytes,
                         void* stream);

/*
 * MatMulNBits (com.microsoft): Y[M,N] = A[M,K] . dequant(B)^T with
 * dequant(B)[n,k] = (q[n,k] - zp[n,k/bs]) * scales[n,k/bs].
 * B: uint8 [N, ceil(K/bs), bs*bits/8] (ORT layout, low nibble first);
 * scales: dtype [N*ceil(K/bs)]; zero_points: NULL (symmetric, zp = 2^(bits-1)),
 * or uint8 packed [N*ceil(ceil(K/bs)/2)] for bits=4, [N*ceil(K/bs)] for bits=8.
 * bits in {4, 8}; block_size in {16, 32, 64, 128}; A, scales and Y share dtype.
 * Replaces: the mlx_quantized_matmul call (rust/src/ops/quant.rs:570-601) reached
 * from matmulnbits_op (quant.rs:986-1130), plus the repack/bias preparation it
 * needs (quant.rs:637-984), which this library does not need: it reads ORT's
 * layout directly.
 */
int ortmi_matmul_nbits(const void* A, const uint8_t* B, const void* scales,
                       const uint8_t* zero_points, void* Y, int64_t M, int64_t N, int64_t K,
                       int64_t bits, int64_t block_size, int32_t dtype, void* stream);

/*
 * MatMulNBits decode step (M = 1, 4-bit, block 32/64/128, fp16/bf16; K up to
 * 16384 in fp16, 10240 in bf16) with its graph neighbours fused in; flags select
 * what is fused:
 *  - ORTMI_FUSE_RMS_NORM: the activation row is first normalised,
 *    a = (x [+ skip]) / sqrt(mean((x [+ skip])^2) + epsilon) * gamma, each
 *    result rounded to dtype as the unfused ops store it; skip is optional, and
 *    residual (optional, needs skip) receives x + skip ([K]).
 *    Replaces: mlx_fast_rms_norm of (Skip)SimplifiedLayerNormalization
 *    (rust/src/ops/norm.rs:164-248) feeding quantized_matmul (quant.rs:570-601).
 *  - ORTMI_FUSE_SWIGLU_PAIRS: B holds N rows interleaved gate/up (row 2i = gate
 *    row i, row 2i+1 = up row i, scales and zero points likewise) and
 *    Y[i] = (g * sigmoid(g)) * u for i < N/2, each op rounded to dtype.
 *    Replaces: the two gate/up quantized_matmul calls and the
 *    Sigmoid/Mul/Mul translation (rust/src/ops/elementwise.rs:928-980).
 * x, skip, gamma, residual: [K]; Y: [N] (or [N/2] with SwiGLU pairs).
 */
enum {
    ORTMI_FUSE_RMS_NORM = 1,
    ORTMI_FUSE_SWIGLU_PAIRS = 2,
};
int ortmi_matmul_nbits_decode_fused(const void* x, const void* skip, const void* gamma,
                                    float epsilon, void* residual, const uint8_t* B,
                                    const void* scales, const uint8_t* zero_points, void* Y,
                                    int64_t N, int64_t K, int64_t block_size, int32_t flags,
                                    int32_t dtype, void* stream);

/*
 * MatMulNBits over interleaved gate/up weight rows (row 2i = gate row i, row
 * 2i+1 = up row i; scales and zero points likewise) with SwiGLU applied in the
 * GEMM epilogue: Y[m, i] = (g * sigmoid(g)) * u, g and u the fp16 matmul outputs,
 * each op rounded to fp16 as the unfused ops store it. A [M, K], Y [M, N/2].
 * fp16 only, 4-bit, block 32/64/128, A and B 16-byte aligned, K % 8 == 0;
 * anything else returns ORTMI_E_INVALID (the caller runs ortmi_matmul_nbits and
 * ortmi_swiglu_pairs instead).
 * Replaces: the gate and up quantized_matmul calls (rust/src/ops/quant.rs:570-601)
 * and the Sigmoid/Mul/Mul translation (rust/src/ops/elementwise.rs:928-980) at
 * prompt lengths M > 1.
 */
int ortmi_matmul_nbits_swiglu_pairs(const void* A, const uint8_t* B, const void* scales,
                                    const uint8_t* zero_points, void* Y, int64_t M, int64_t N,
                                    int64_t K, int64_t block_size, int32_t dtype, void* stream);

/*
 * MatMulNBits decode step (M = 1) whose activation row is the output of the
 * one-token GroupQueryAttention still held as split partials (written by
 * ortmi_group_query_attention_decode_partials): partials [K / head_size heads]
 * [splits][head_size + 2] fp32 (o[head_size], max, sum), merged per head as
 * a = (sum_i e^(m_i - M) o_i) / (sum_i e^(m_i - M) l_i), M = max_i m_i, rounded
 * to dtype, then the GEMV. K = heads * head_size (batch 1). fp16/bf16 only.
 * Replaces: the GQA output write (rust/src/ops/attention.rs:910-920) and the
 * o_proj quantized_matmul (rust/src/ops/quant.rs:570-601) reading it back.
 */
int ortmi_matmul_nbits_decode_merge(const float* partials, int64_t splits, int64_t head_size,
                                    const uint8_t* B, const void* scales,
                                    const uint8_t* zero_points, void* Y, int64_t N, int64_t K,
                                    int64_t block_size, int32_t dtype, void* stream);

/*
 * Int4 decoder decode step as one launch: the whole one-token step of a
 * Llama-style decoder graph (embedding Gather; per layer
 * (Skip)SimplifiedLayerNormalization, q/k/v MatMulNBits, GroupQueryAttention over
 * a shared KV cache with in-op RoPE, o_proj MatMulNBits,
 * SkipSimplifiedLayerNormalization, gate/up MatMulNBits with SwiGLU
 * (Sigmoid/Mul/Mul), down MatMulNBits; final SkipSimplifiedLayerNormalization;
 * lm_head MatMulNBits) plus the greedy argmax of the logits.
 * Forms: fp16, 4-bit symmetric weights (no zero points), block 32, head size
 * 64, 96 or 128, non-interleaved rotary (or none), at most 8 query heads per KV
 * head, hidden and num_heads * head_size multiples of 32 up to 3072,
 * intermediate a multiple of 32 up to 10240, and projection rows that fit the
 * per-workgroup share (QKV: at most two groups of 4 rows per wave, down_proj: at
 * most two rows per wave of the projection workgroups; the key splits per head
 * shrink until the rows fit). Other forms return ORTMI_E_INVALID before any
 * launch (the caller runs the graph op by op).
 * Weights keep the MatMulNBits layout [N, K/32, 16] with fp16 scales [N * K/32];
 * qkv_weight holds the q rows, then the k rows, then the v rows of one merged
 * projection; gate_up_weight interleaves gate row i (row 2i) and up row i
 * (row 2i+1). k_cache / v_cache [1, kv_num_heads, kv_capacity, head_size] are past
 * and present at once: the step writes the new row at total - 1 in place.
 * `layers` is a device array of `dims->layers` records. input_id (int64 [1]) and
 * total_sequence_length (int32 [1]) are device memory read by the kernel, so a
 * step needs no host round trip; logits [vocab] fp16 and next_id (int64, the
 * first index of the largest logit, NaN never wins; device or host-pinned
 * memory, written once at the end of the step) are written. `status`
 * (optional; device or host-pinned memory) receives 0 on success, 1 if a wait
 * between the step's workgroups saw no data for 100 ms (the results are then
 * invalid), 2 if the token id was out of range (row 0 was used), 3 if
 * total_sequence_length is outside [1, kv_capacity] or past the rotary table
 * (nothing computed); it is left unwritten by a launch the host aborted before
 * it started (below), so a caller that sets it to -1 before each step sees every
 * step that did not complete. The workspace
 * (ortmi_decoder_decode_step_workspace_size bytes, 256-byte aligned) must be
 * zero-filled before its first use and then passed unchanged to every step;
 * steps sharing a workspace must run in order on one stream. Its first 8 bytes
 * count started workgroups (a 64-bit integer; launch index = count / grid, the
 * grid being the device's CU count rounded down to a multiple of 8), and the
 * 32-bit word at byte 128 aborts the launch whose index + 1 it holds: that
 * launch reads and writes nothing. A step that is not completed leaves the KV
 * row at total - 1 possibly written; running the step again (by this call or op
 * by op) rewrites it with the same values. embed, the gammas and the cos/sin
 * caches must be 16-byte aligned. dims->cooperative selects the launch: 1 a
 * cooperative launch (every workgroup resident, guaranteed); 0 a plain launch of
 * the same grid, about 30 us cheaper per step, whose workgroups are all resident
 * when no other work holds a CU of the device; when one cannot start, the launch
 * ends with status 1 after a 100 ms wait and the step must be run again (by this
 * call with cooperative = 1, or op by op).
 * Replaces: the compiled decode path of the reference EP, a shapeless
 * mlx_compile trace of the decode graph evaluated once per token
 * (rust/src/compiled.rs:503-822, rust/src/engine.rs:417, 1720-1736), over the
 * op translations of rust/src/ops/quant.rs:570-601, attention.rs:556-952 and
 * norm.rs:164-248.
 */
typedef struct OrtmiDecoderLayer {
    const uint8_t* qkv_weight;
    const void* qkv_scales;
    const void* ln1_gamma;     /* norm before the attention */
    float ln1_epsilon;
    int32_t reserved0;
    const uint8_t* o_weight;
    const void* o_scales;
    const void* ln2_gamma;     /* norm before the MLP */
    float ln2_epsilon;
    int32_t reserved1;
    const uint8_t* gate_up_weight;
    const void* gate_up_scales;
    const uint8_t* down_weight;
    const void* down_scales;
    void* k_cache;
    void* v_cache;
} OrtmiDecoderLayer;

typedef struct OrtmiDecoderDims {
    int32_t layers, hidden, num_heads, kv_num_heads, head_size, intermediate, vocab;
    int32_t kv_capacity, max_position, rotary_half, rotary_interleaved, block_size, dtype;
    float scale; /* 0: 1/sqrt(head_size) */
    /* 0: a plain launch of one workgroup per CU (every workgroup resident when no
     * other work holds a CU); 1: a cooperative launch, which guarantees it. */
    int32_t cooperative;
} OrtmiDecoderDims;

size_t ortmi_decoder_decode_step_workspace_size(const OrtmiDecoderDims* dims);
int ortmi_decoder_decode_step(const OrtmiDecoderLayer* layers, const OrtmiDecoderDims* dims,
                              const void* embed, int64_t embed_rows, const int64_t* input_id,
                              const int32_t* total_sequence_length, const void* cos_cache,
                              const void* sin_cache, const void* final_gamma,
                              float final_epsilon, const uint8_t* lm_weight,
                              const void* lm_scales, void* logits, int64_t* next_id,
                              int32_t* status, void* workspace, size_t workspace_bytes,
                              void* stream);

/*
 * GroupQueryAttention (com.microsoft), decode and prefill, with in-op RoPE.
 * query [B,S,H*hd] (or packed [B,S,(H+2*KV)*hd] when key == value == NULL),
 * key/value [B,S,KV*hd]; past_key/past_value [B,KV,past_cap,hd].
 * valid_past = total_sequence_length - S (one value for the batch); the
 * shared-buffer contract applies when past_cap > valid_past: present_* are
 * [B,KV,past_cap,hd] (they may alias past_*, then only the S new rows are
 * written); otherwise the growing contract: present_* are [B,KV,past_cap+S,hd].
 * cos_cache/sin_cache [max_pos, rotary_half] (NULL when do_rotary = 0), in dtype.
 * output [B,S,H*hd]. scale = 0 means 1/sqrt(hd). hd is 64, 96 or 128 (other head
 * sizes, fp32, attention_bias and QK-norm: ortmi_group_query_attention_ex).
 * Replaces: group_query_attention_op (rust/src/ops/attention.rs:556-952): the
 * two mlx_fast_rope calls (attention.rs:671-708), the KV concat /
 * slice_update (attention.rs:881-908) and mlx_fast_scaled_dot_product_attention
 * (attention.rs:111-135, 264-285).
 */
size_t ortmi_group_query_attention_workspace_size(int64_t batch, int64_t seq_len,
                                                  int64_t num_heads, int64_t head_size,
                                                  int64_t total_kv);
int ortmi_group_query_attention(const void* query, const void* key, const void* value,
                                const void* past_key, const void* past_value,
                                int64_t past_cap, int32_t total_sequence_length,
                                const void* cos_cache, const void* sin_cache,
                                int64_t rotary_half, int64_t max_pos,
                                void* output, void* present_key, void* present_value,
                                int64_t batch, int64_t seq_len, int64_t num_heads,
                                int64_t kv_num_heads, int64_t head_size, float scale,
                                int32_t rotary_interleaved, int32_t dtype, void* workspace,
                                size_t workspace_bytes, void* stream);

/*
 * GroupQueryAttention with the optional inputs of the 11- and 16-input forms,
 * for fp32, fp16 and bf16, head_size a multiple of 16 up to 256. Arguments and
 * KV contract as ortmi_group_query_attention, plus:
 *  - q_norm_weight / k_norm_weight [head_size] (inputs 14/15, both or neither,
 *    in dtype): q and the new k are RMS-normalised per head with qk_norm_epsilon
 *    before RoPE (rust/src/ops/attention.rs:663-670, claim 1698-1720);
 *  - attention_bias (input 10, NULL when absent, in dtype), contiguous
 *    [bias_batch, bias_heads, bias_rows, bias_cols] with bias_batch in {1, batch},
 *    bias_heads in {1, num_heads}, bias_rows >= seq_len and bias_cols >=
 *    valid_past + seq_len: entry [b, h, s, j] is added to scale * q.k of key j
 *    and the causal mask still applies (attention.rs:256-285, claim 1637-1657).
 * The workspace holds ortmi_group_query_attention_ex_workspace_size bytes.
 * Replaces: the same reference op as ortmi_group_query_attention, for the forms
 * whose rms_norm / array-mask SDPA calls (attention.rs:663-670, 264-285) the fused
 * kernels do not cover.
 */
size_t ortmi_group_query_attention_ex_workspace_size(int64_t batch, int64_t seq_len,
                                                     int64_t num_heads, int64_t head_size);
int ortmi_group_query_attention_ex(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, int32_t total_sequence_length,
    const void* cos_cache, const void* sin_cache, int64_t rotary_half, int64_t max_pos,
    const void* q_norm_weight, const void* k_norm_weight, float qk_norm_epsilon,
    const void* attention_bias, int64_t bias_batch, int64_t bias_heads, int64_t bias_rows,
    int64_t bias_cols, void* output, void* present_key, void* present_value, int64_t batch,
    int64_t seq_len, int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* workspace, size_t workspace_bytes,
    void* stream);

/*
 * GroupQueryAttention with sliding_window_cache = 1: past_key / past_value
 * [batch, kv_num_heads, past_cap, head_size] are a compacting cache. Per sequence
 * b, p = max(seqlens_k[b] + 1 - seq_len, 0) tokens precede the new ones and the
 * cache holds the last cache_end(p) of them in rows [0, cache_end(p)), where
 * cache_end(n) = n for n <= past_cap, else n - gap * ceil((n - past_cap) / gap)
 * with gap = past_cap - local_window_size + 1 (the cache drops its oldest gap rows
 * whenever it is full). Query s of sequence b, at position p + s (its RoPE
 * position too), attends the positions (p + s - local_window_size, p + s].
 * present_key / present_value [batch, kv_num_heads, past_cap, head_size] receive
 * the last cache_end(p + seq_len) rows (new K rows RoPE'd), zeros after; they may
 * be the past buffers themselves. seqlens_k is device int32 [batch]; RoPE
 * positions past the cos/sin rows read the last row. q_norm_weight /
 * k_norm_weight, dtypes and head sizes as ortmi_group_query_attention_ex; no
 * attention_bias (the reference declines the pair). The workspace holds
 * ortmi_group_query_attention_sliding_workspace_size bytes.
 * Replaces: the sliding-cache branch of group_query_attention_op
 * (rust/src/ops/attention.rs:725-880) and its causal_window_mask (191-219).
 */
size_t ortmi_group_query_attention_sliding_workspace_size(int64_t batch, int64_t seq_len,
                                                          int64_t num_heads,
                                                          int64_t kv_num_heads,
                                                          int64_t head_size, int64_t past_cap);
int ortmi_group_query_attention_sliding(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, const int32_t* seqlens_k, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, const void* q_norm_weight,
    const void* k_norm_weight, float qk_norm_epsilon, int64_t local_window_size, void* output,
    void* present_key, void* present_value, int64_t batch, int64_t seq_len, int64_t num_heads,
    int64_t kv_num_heads, int64_t head_size, float scale, int32_t rotary_interleaved,
    int32_t dtype, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ortmi_group_query_attention without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). It has no counterpart in the
 * reference. Arguments and results are those of ortmi_group_query_attention;
 * the workspace is a fixed scratch array inside this library, one per GPU
 * (ortmi_group_query_attention_noalloc_max_workspace() bytes, 32 MiB), held
 * until the process ends. A call whose
 * ortmi_group_query_attention_workspace_size(batch, seq_len, num_heads,
 * head_size, valid_past + seq_len) exceeds it returns ORTMI_E_WORKSPACE before
 * any launch. The call allocates nothing. Every call on one GPU shares that
 * GPU's scratch, so calls that overlap on one GPU (concurrent streams or
 * threads) race; calls ordered on one stream do not.
 */
size_t ortmi_group_query_attention_noalloc_max_workspace(void);
int ortmi_group_query_attention_noalloc(
    const void* query, const void* key, const void* value, const void* past_key,
    const void* past_value, int64_t past_cap, int32_t total_sequence_length,
    const void* cos_cache, const void* sin_cache, int64_t rotary_half, int64_t max_pos,
    void* output, void* present_key, void* present_value, int64_t batch, int64_t seq_len,
    int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* stream);

/*
 * One-token GroupQueryAttention decode step over a fixed-capacity shared KV
 * buffer, in a form that can be captured into a HIP graph and replayed across
 * steps: total_sequence_length is read from device memory by the kernels, and
 * the launch shape depends only on kv_cap. kv_key/kv_value [B,KV,kv_cap,hd] are
 * both past and present (the new row is written at total-1, in place). Results
 * equal ortmi_group_query_attention's for seq_len = 1 under the shared-buffer
 * contract. The caller guarantees 1 <= total <= kv_cap (and total <= max_pos
 * with rotary); the kernels clamp the row index into the buffers regardless.
 * Workspace: ortmi_group_query_attention_workspace_size(B, 1, H, hd, kv_cap).
 * Returns ORTMI_E_INVALID for forms without a capturable kernel (more than 8
 * query heads per KV head, unaligned tensors, rotary half not a multiple of 8).
 * Replaces: the compiled-decode fast path (rust/src/engine.rs:417, 1720-1736),
 * where a shapeless mlx_compile trace reads valid_past from a tensor so one
 * compiled closure serves every decode step.
 */
int ortmi_group_query_attention_decode_capturable(
    const void* query, const void* key, const void* value, void* kv_key, void* kv_value,
    int64_t kv_cap, const int32_t* total_sequence_length_device, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, void* output, int64_t batch,
    int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* workspace, size_t workspace_bytes,
    void* stream);

/*
 * The one-token step of ortmi_group_query_attention_decode_capturable, leaving
 * the attention output as split partials for ortmi_matmul_nbits_decode_merge
 * (the o_proj consumer) instead of merging them: partials [batch * num_heads]
 * [splits][head_size + 2] fp32 (16-byte aligned), splits =
 * ortmi_group_query_attention_decode_splits(batch, num_heads, kv_num_heads,
 * head_size, kv_cap), chosen so that the partials of all heads stay within what
 * the merging GEMV stages (8192 floats); 0 (and ORTMI_E_INVALID from the step,
 * before any write) when even one split per head does not fit. No workspace.
 * The KV append is the same.
 * Replaces: as ortmi_group_query_attention_decode_capturable, minus the output
 * write (rust/src/ops/attention.rs:910-920), which the consumer folds in.
 */
int64_t ortmi_group_query_attention_decode_splits(int64_t batch, int64_t num_heads,
                                                  int64_t kv_num_heads, int64_t head_size,
                                                  int64_t kv_cap);
int ortmi_group_query_attention_decode_partials(
    const void* query, const void* key, const void* value, void* kv_key, void* kv_value,
    int64_t kv_cap, const int32_t* total_sequence_length_device, const void* cos_cache,
    const void* sin_cache, int64_t rotary_half, int64_t max_pos, float* partials, int64_t batch,
    int64_t num_heads, int64_t kv_num_heads, int64_t head_size, float scale,
    int32_t rotary_interleaved, int32_t dtype, void* stream);

/*
 * PagedAttention (com.microsoft), mixed prefill + decode over a block-paged KV
 * cache. query [T,H*hd], key [T,KV*hd], value [T,KV*vhd] (value == NULL and
 * value_cache == NULL selects the LATENT layout: values are the first vhd dims
 * of the keys); key_cache [num_blocks, block_size, KV, hd], value_cache
 * [num_blocks, block_size, KV, vhd], updated in place. cum_seqlens [batch+1],
 * past_seqlens [batch], block_table [batch, max_blocks] and slot_mapping [T]
 * (optional, slot < 0 skips the write) are int32 device tensors: nothing is read
 * back to the host. max_context is a host upper bound on past + new tokens of
 * every sequence (max_blocks * block_size always is one); keys at positions
 * max_context and beyond are not attended, and past_seqlens is read clamped to
 * [0, max_context]. dtype fp32, fp16 or bf16; head_size a multiple of 16 up to
 * 256 (fp16/bf16 with head 64/128 run the multi-token tiles on the matrix cores
 * and the single-token decode kernel; every other form one VALU workgroup per
 * (token, head) row). A token's
 * sequence range is cum_seqlens clamped to [0, num_tokens). cos/sin caches are
 * [rotary_max_pos, rotary_half]. head_sink [H],
 * q_norm_weight/k_norm_weight [hd] optional. output [T,H*vhd]. Malformed control
 * tensors (block ids or positions out of range) never cause out-of-bounds
 * accesses: such keys are masked and such writes skipped.
 * Replaces: paged_attention_op (rust/src/ops/attention.rs:2495-2744), which
 * syncs the control tensors to the host and loops over sequences with MLX
 * take/scatter/concat and fp32 SDPA.
 */
size_t ortmi_paged_attention_workspace_size(int64_t num_tokens, int64_t batch,
                                            int64_t num_heads, int64_t kv_num_heads,
                                            int64_t head_size, int64_t v_head_size,
                                            int64_t max_context);
int ortmi_paged_attention(const void* query, const void* key, const void* value,
                          void* key_cache, void* value_cache, int64_t num_blocks,
                          int64_t block_size, const int32_t* cum_seqlens,
                          const int32_t* past_seqlens, const int32_t* block_table,
                          int64_t batch, int64_t max_blocks, int64_t num_tokens,
                          int64_t max_context, const void* cos_cache, const void* sin_cache,
                          int64_t rotary_half, int64_t rotary_max_pos,
                          int32_t rotary_interleaved, int64_t rotary_offset, const int32_t* slot_mapping,
                          const void* head_sink, const void* q_norm_weight,
                          const void* k_norm_weight, float qk_norm_eps, void* output,
                          int64_t num_heads, int64_t kv_num_heads, int64_t head_size,
                          int64_t v_head_size, float scale, int32_t dtype, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * RotaryEmbedding (com.microsoft / ai.onnx), standalone.
 * x: rank-3 [B,S,NH*hd] (is_bnsd = 0) or rank-4 [B,NH,S,hd] (is_bnsd = 1).
 * Position forms (rust/src/ops/attention.rs:1288-1315, 1337-1400):
 *   position_ids == NULL: cos/sin are per-token [B*S, half] rows;
 *   pos_is_offset = 1: position_ids is int64 [1], token (b,s) uses row offset+s;
 *   otherwise position_ids is int64 [B,S].
 * cos/sin are [max_pos, rotary_half]. Rotates dims [0, 2*rotary_half) of each
 * head; the rest pass through.
 * Replaces: rotary_embedding_op (attention.rs:1317-1411) / mlx_fast_rope.
 */
int ortmi_rotary_embedding(const void* x, const int64_t* position_ids, int32_t pos_is_offset,
                           const void* cos_cache, const void* sin_cache, int64_t max_pos, void* y,
                           int64_t batch, int64_t seq_len, int64_t num_heads,
                           int64_t head_size, int64_t rotary_half, int32_t is_bnsd,
                           int32_t interleaved, int32_t dtype, void* stream);

/*
 * GatherBlockQuantized (com.microsoft), 4-bit, gather_axis 0, quantize_axis 1:
 * out[i, k] = (q[row_i, k] - zp[row_i, k / block]) * scales[row_i, k / block],
 * computed in fp32 and rounded once to dtype. data [rows, D/2] uint8 (two codes
 * per byte, low nibble first), scales [rows, ceil(D/block)] in dtype (= the
 * output dtype), zero_points [rows, ceil(ceil(D/block)/2)] packed int4 (low nibble
 * = even block) or NULL (8). indices [num_indices] int32 or int64 (negative ids
 * count from the end; ids outside [-rows, rows) give zero rows). output
 * [num_indices, D]. block_size >= 16.
 * Replaces: gather_block_quantized_op (rust/src/ops/quant.rs:1134-1199) and the
 * claim checks of quant.rs:1713-1749.
 */
int ortmi_gather_block_quantized(const uint8_t* data, const void* scales,
                                 const uint8_t* zero_points, const void* indices,
                                 int32_t indices_are_int64, void* output, int64_t num_indices,
                                 int64_t rows, int64_t D, int64_t block_size, int64_t bits,
                                 int32_t dtype, void* stream);

/*
 * SimplifiedLayerNormalization / SkipSimplifiedLayerNormalization
 * (com.microsoft) and RMSNormalization: r = x (+ skip) (+ bias);
 * y = r / sqrt(mean(r^2) + eps) * gamma over the last axis of length D.
 * skip, bias and residual_out are optional (NULL).
 * Replaces: mlx_fast_rms_norm via simplified_layer_norm_op / skip_rms_norm_op /
 * rms_norm_op (rust/src/ops/norm.rs:164-248).
 */
int ortmi_rms_norm(const void* x, const void* skip, const void* bias, const void* gamma,
                   void* y, void* residual_out, int64_t rows, int64_t D, float eps,
                   int32_t dtype, void* stream);

/*
 * Decoder glue claimed with the hot path so the whole int4 decoder graph runs on
 * the device (rust/src/ops/elementwise.rs:928-980, rust/src/ops/shape.rs:2453).
 *  - ortmi_gather_rows: Gather along axis 0 of a [V, D] table by int64 ids
 *    (negative ids count from the end, out of range is reported via the
 *    returned status only when checked on the host by the caller).
 *  - ortmi_swiglu: out = (g * sigmoid(g)) * u, each op rounded to dtype as the
 *    Sigmoid/Mul/Mul graph does.
 *  - ortmi_swiglu_pairs: the same over interleaved gate/up columns, y [rows, 2P]
 *    (column 2i gate, 2i+1 up) -> out [rows, P]; the prefill side of the
 *    SwiGLU-pairs fusion of ortmi_matmul_nbits_decode_fused.
 *  - ortmi_binary: elementwise Add (op 0) / Mul (op 1) / Sub (op 2) of
 *    same-shape tensors.
 *  - ortmi_sigmoid: elementwise Sigmoid.
 *  - ortmi_argmax_rows: int64 index of the max of each row (first on ties; NaN
 *    never wins). With a workspace of ortmi_argmax_rows_workspace_size bytes,
 *    long rows are reduced by many workgroups in two passes; with workspace =
 *    NULL one workgroup scans each row. Greedy decoding takes it over the last
 *    logits row (the reference's callers do this on the host after Compute).
 *  - ortmi_argmax_axis: ArgMax over any axis, x viewed as [outer, dim, inner],
 *    out [outer, inner] int64; select_last_index = 1 gives the last index on
 *    ties (0 the first); NaN never wins, an all-NaN slice gives 0. Replaces
 *    argminmax / argmax_op (rust/src/ops/reduction.rs:239-278; claim
 *    reduction.rs:582-630) for the axes and tie rule ortmi_argmax_rows does not
 *    cover.
 *  - ortmi_cast: f32 <-> f16 <-> bf16.
 */
int ortmi_gather_rows(const void* table, const int64_t* ids, void* out, int64_t num_ids,
                      int64_t vocab, int64_t D, int32_t dtype, void* stream);
int ortmi_swiglu(const void* gate, const void* up, void* out, int64_t n, int32_t dtype,
                 void* stream);
int ortmi_swiglu_pairs(const void* y, void* out, int64_t rows, int64_t pairs, int32_t dtype,
                       void* stream);
int ortmi_binary(int32_t op, const void* a, const void* b, void* out, int64_t n,
                 int32_t dtype, void* stream);
int ortmi_sigmoid(const void* x, void* out, int64_t n, int32_t dtype, void* stream);
size_t ortmi_argmax_rows_workspace_size(int64_t rows, int64_t cols);
int ortmi_argmax_rows(const void* x, int64_t* out, int64_t rows, int64_t cols, int32_t dtype,
                      void* workspace, size_t workspace_bytes, void* stream);
int ortmi_argmax_axis(const void* x, int64_t* out, int64_t outer, int64_t dim, int64_t inner,
                      int32_t select_last_index, int32_t dtype, void* stream);
int ortmi_cast(const void* x, int32_t src_dtype, void* y, int32_t dst_dtype, int64_t n,
               void* stream);

#ifdef __cplusplus
}
#endif
#endif
