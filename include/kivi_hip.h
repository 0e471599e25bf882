/*
 * kivi_hip.h -- C ABI of libkivi_hip.so, the MI355X (gfx950) KIVI KV-cache
 * hot path.
 *
 * Every function takes raw device pointers, element counts and a HIP stream
 * (hipStream_t passed as void*; NULL = the default stream), launches its work
 * on that stream and returns without waiting: 0 on success, a KIVI_ERR_* code
 * otherwise, with a message available from kivi_last_error() (thread-local).
 * No function allocates device memory unless its comment says so, and none
 * throws across the ABI.  The caller owns every buffer (the reference's
 * "caller allocates every output" contract, src/csrc/ops/kv_cache_ops.cpp:179-237).
 *
 * Reference interface replaced by each entry point is cited beside it
 * (paths relative to the reference checkout).
 */
#ifndef KIVI_HIP_H
#define KIVI_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KIVI_HIP_ABI_VERSION 7

#define KIVI_OK 0
#define KIVI_ERR_INVALID_ARGUMENT 1
#define KIVI_ERR_LAUNCH 2
#define KIVI_ERR_RUNTIME 3
#define KIVI_ERR_UNSUPPORTED 4

/* ---- runtime glue --------------------------------------------------------
 * Replaces src/csrc/include/kivi/common.hpp:26-61 (queue selection: here the
 * caller's stream) and src/csrc/include/kivi/event.hpp:16-31 (KiviEvent). */
const char* kivi_last_error(void);
void kivi_clear_error(void);
int kivi_abi_version(void);
int kivi_stream_synchronize(void* stream);
/* Records an event on `stream`; *event_out receives an owned handle. */
int kivi_event_record(void* stream, void** event_out);
/* Blocks until the event completes; reports asynchronous device errors
 * (KiviEvent.wait, event.hpp:25). */
int kivi_event_wait(void* event);
/* 1 = complete, 0 = pending, negative = -error code. */
int kivi_event_query(void* event);
int kivi_event_destroy(void* event);

/* ---- 2-bit codec ---------------------------------------------------------
 * Flat groups of `group_size` contiguous floats; group g's packed bytes sit at
 * g*group_size/4 (element 4j+k -> byte j bits 2k..2k+1), scales[g] =
 * (max-min)/3 + 1e-10, zeros[g] = min. */

/* quantize_keys_per_channel, src/csrc/kernels/quantize_kernels.hpp /
 * quantize_kernels.cpp:24-67; input [.., Seq] f32 with Seq groups per channel
 * row, num_channels = number of groups (kv_cache_ops.cpp:30). */
int kivi_quantize_keys_per_channel(const float* input, uint8_t* output, float* scales,
                                   float* zeros, int64_t num_channels, int32_t group_size,
                                   void* stream);

/* quantize_values_per_token, quantize_kernels.cpp:69-120; input
 * [num_tokens, head_dim] f32, head_dim % group_size == 0. */
int kivi_quantize_values_per_token(const float* input, uint8_t* output, float* scales,
                                   float* zeros, int64_t num_tokens, int32_t head_dim,
                                   int32_t group_size, void* stream);

/* dequantize_keys_per_channel, src/csrc/kernels/dequantize_kernels.cpp:32-77. */
int kivi_dequantize_keys_per_channel(const uint8_t* input, const float* scales,
                                     const float* zeros, float* output, int64_t num_channels,
                                     int32_t group_size, void* stream);

/* dequantize_values_per_token, dequantize_kernels.cpp:79-124; num_groups =
 * scales.numel() (kv_cache_ops.cpp:118). */
int kivi_dequantize_values_per_token(const uint8_t* input, const float* scales,
                                     const float* zeros, float* output, int64_t num_groups,
                                     int32_t group_size, void* stream);

/* quant_dequant_roundtrip_keys, src/csrc/kernels/roundtrip_kernels.cpp:14-48:
 * output is bit-identical to quantize + dequantize of the same input. */
int kivi_quant_dequant_roundtrip_keys(const float* input, float* output,
                                      int64_t num_channels, int32_t group_size,
                                      void* stream);

/* quant_dequant_roundtrip_values, roundtrip_kernels.cpp:50-91. */
int kivi_quant_dequant_roundtrip_values(const float* input, float* output,
                                        int64_t num_tokens, int32_t head_dim,
                                        int32_t group_size, void* stream);

/* The six ops above, each also returning in *event_out a new event handle
 * (owned by the caller: kivi_event_wait / kivi_event_query /
 * kivi_event_destroy) that is the completion event of the op's own kernel
 * launch: the *_async ops of the reference, whose KiviEvent wraps the
 * submitted kernel's sycl::event (kv_cache_ops.cpp:245-303, event.hpp:16-31).
 * No marker is queued after the kernel, unlike kivi_event_record.  On error
 * *event_out is NULL. */
int kivi_quantize_keys_per_channel_ev(const float* input, uint8_t* output, float* scales,
                                      float* zeros, int64_t num_channels, int32_t group_size,
                                      void* stream, void** event_out);
int kivi_quantize_values_per_token_ev(const float* input, uint8_t* output, float* scales,
                                      float* zeros, int64_t num_tokens, int32_t head_dim,
                                      int32_t group_size, void* stream, void** event_out);
int kivi_dequantize_keys_per_channel_ev(const uint8_t* input, const float* scales,
                                        const float* zeros, float* output,
                                        int64_t num_channels, int32_t group_size, void* stream,
                                        void** event_out);
int kivi_dequantize_values_per_token_ev(const uint8_t* input, const float* scales,
                                        const float* zeros, float* output, int64_t num_groups,
                                        int32_t group_size, void* stream, void** event_out);
int kivi_quant_dequant_roundtrip_keys_ev(const float* input, float* output,
                                         int64_t num_channels, int32_t group_size,
                                         void* stream, void** event_out);
int kivi_quant_dequant_roundtrip_values_ev(const float* input, float* output,
                                           int64_t num_tokens, int32_t head_dim,
                                           int32_t group_size, void* stream,
                                           void** event_out);

/* ---- HBM-resident packed store --------------------------------------------
 * Replaces KiviCache._flush_group (src/kivi_sycl/cache/manager.py:309-374):
 * quantises the `group_size_k` oldest tokens of the residual ring of every
 * (batch, kv-head) into chunk `chunk_index` of the packed store, on the
 * device, without host copies.  Per (b, kv-head):
 *   k_res, v_res    [res_capacity][head_dim] ring, 16-byte aligned, of
 *                   element type res_dtype (0 f32, 1 bf16, 2 f16; 16-bit
 *                   values are widened exactly, so a 16-bit ring holding a
 *                   half-precision model's K/V gives the results of an f32
 *                   ring holding the same values); token t of the window
 *                   sits at slot (res_start + t) % res_capacity
 *   k_codes, v_codes [chunk_capacity][G*head_dim/4] u8 per chunk, in the code
 *                   layout kivi_store_code_layout() reports:
 *                   0 (plain): keys [G][D/4] (byte (t,i) = channels 4i..4i+3 of
 *                     token t, channel 4i+k at bits 2k), values [D][G/4] (byte
 *                     (d,j) = tokens 4j..4j+3 of channel d, token 4j+k at bits 2k);
 *                   1 (matrix-core operand order): [64 lanes][G*D/1024 dwords]
 *                     holding v_mfma_f32_16x16x32_bf16 B operands -- key tile
 *                     ks*(G/16)+nb: lane l element j = token 16nb+l%16, channel
 *                     32ks+8(l/16)+j; value tile kt*(D/16)+nb: lane l element j
 *                     = token 32kt+8(l/16)+j, channel 16nb+l%16; tiles 2w and
 *                     2w+1 share dword w, element j of tile 2w+m at bit
 *                     8m+2(j/2)+16(j%2).
 *   k_scale, k_zero [chunk_capacity][head_dim] f32 (per channel per chunk)
 *   v_scale, v_zero [chunk_capacity][head_dim/group_size_v][G] f32
 * Codes, scales and zeros equal quantize_keys on the chunk's [D, G] transpose
 * and quantize_values on its [G, D] rows; only their order differs.  If
 * k_hist/v_hist are non-null ([hist_capacity][head_dim] f32 per (b, kv-head))
 * the dequantised tokens are also written at rows chunk_index*G .. +G-1
 * (bit-identical to the round-trip ops, manager.py:337-345).  Requires
 * group_size_k * head_dim <= 65536. */
int kivi_store_flush(const void* k_res, const void* v_res, int32_t res_dtype,
                     uint8_t* k_codes, float* k_scale, float* k_zero, uint8_t* v_codes, float* v_scale,
                     float* v_zero, float* k_hist, float* v_hist, int64_t hist_capacity,
                     int32_t batch, int32_t kv_heads, int32_t head_dim,
                     int32_t group_size_k, int32_t group_size_v, int32_t res_capacity,
                     int32_t res_start, int32_t chunk_capacity, int32_t chunk_index,
                     void* stream);

/* Quantise n_chunks consecutive chunks in one launch (grid: (b, kv-head) x
 * chunk) from the run of tokens formed by the residual window (res_len tokens
 * of the ring, starting at slot res_start) followed by new_tokens new tokens
 * that have not been copied anywhere: element (b, h, t, d) of k_new/v_new is
 * at b*new_batch_stride + h*new_head_stride + t*new_token_stride + d (in
 * elements of new_dtype: 0 f32, 1 bf16, 2 f16; both tensors share the
 * strides).  Chunk j takes tokens [j*G, (j+1)*G) of that run and is written
 * as chunk chunk_index + j in the layout of kivi_store_flush (same codes,
 * scales, zeros and history rows).  bf16/f16 inputs are widened exactly.
 * Replaces the flush loop of KiviCache.add_tokens (manager.py:242-249) and the
 * host-side transpose of each chunk (manager.py:332-334): a prompt of P
 * tokens is quantised by one launch.  The caller then keeps the tokens after
 * the last chunk (in the ring, and the new tokens past n_chunks*G - res_len).
 * Requires n_chunks*G <= res_len + new_tokens and group_size_k * head_dim <=
 * 65536. */
int kivi_store_flush_chunks(const void* k_res, const void* v_res, int32_t res_dtype,
                            const void* k_new, const void* v_new, int32_t new_dtype, int64_t new_batch_stride,
                            int64_t new_head_stride, int64_t new_token_stride,
                            int32_t new_tokens, uint8_t* k_codes, float* k_scale,
                            float* k_zero, uint8_t* v_codes, float* v_scale, float* v_zero,
                            float* k_hist, float* v_hist, int64_t hist_capacity,
                            int32_t batch, int32_t kv_heads, int32_t head_dim,
                            int32_t group_size_k, int32_t group_size_v, int32_t res_capacity,
                            int32_t res_start, int32_t res_len, int32_t chunk_capacity,
                            int32_t chunk_index, int32_t n_chunks, void* stream);

/* Append new_tokens tokens to the residual ring of every (b, kv-head): token
 * t of k_new/v_new (element (b, h, t, d) at b*new_batch_stride +
 * h*new_head_stride + t*new_token_stride + d, in elements of new_dtype: 0
 * f32, 1 bf16, 2 f16) goes to ring slot (slot + t) % res_capacity.  An f32
 * ring (res_dtype 0) takes any new_dtype, widened exactly; a bf16 or f16 ring
 * takes its own type only, copied bit for bit.  K and V in one launch.  Replaces the residual
 * append of KiviCache.add_tokens (manager.py:226-231, a torch.cat of the
 * fp32 residual); the caller keeps the window's start and length. */
int kivi_store_append(const void* k_new, const void* v_new, int32_t new_dtype,
                      int64_t new_batch_stride, int64_t new_head_stride,
                      int64_t new_token_stride, int32_t new_tokens, void* k_res, void* v_res,
                      int32_t res_dtype, int32_t batch, int32_t kv_heads, int32_t head_dim, int32_t res_capacity,
                      int32_t slot, void* stream);

/* kivi_store_append for n_layers layers of one model in as few launches as
 * possible (16 layers per launch): layer l's new tokens k_new[l]/v_new[l]
 * with element strides new_strides[3l..3l+2] (batch, head, token) go to its
 * ring k_res[l]/v_res[l] from slot slots[l].  The shapes, element types and
 * ring capacity are shared; host arrays of n_layers entries.  Replaces the
 * per-layer residual append of KiviCache.add_tokens's layer loop
 * (manager.py:187-231: each layer's new K/V appended to its residual), one
 * launch per step instead of one per layer. */
int kivi_store_append_layers(int32_t n_layers, const void* const* k_new, const void* const* v_new,
                             const int64_t* new_strides, int32_t new_dtype, int32_t new_tokens,
                             void* const* k_res, void* const* v_res, int32_t res_dtype,
                             int32_t batch, int32_t kv_heads, int32_t head_dim,
                             int32_t res_capacity, const int32_t* slots, void* stream);

/* Code layout of a store with these shapes: 1 (matrix-core operand order)
 * when head_dim is 64, 128 or 256, group_size_k is 32 or 64 and
 * group_size_v is a multiple of 32 dividing head_dim; 0 (plain) otherwise.
 * No reference counterpart (the reference keeps no packed store). */
int kivi_store_code_layout(int32_t head_dim, int32_t group_size_k, int32_t group_size_v);

/* ---- fused packed-KV decode attention -------------------------------------
 * No reference counterpart (the reference runs HF attention on the CPU over
 * the dequantised history, manager.py:251-290; its stated math is
 * tests/integration/test_attention_fix.py:40-43).  For q [batch][q_heads]
 * [head_dim] f32, computes out [batch][q_heads][head_dim] =
 *   softmax(q . [K_hat ; K_res]^T * softmax_scale) . [V_hat ; V_res]
 * over the first num_chunks chunks of the packed store (layout above) and the
 * res_len residual tokens (ring of element type res_dtype, as for
 * kivi_store_flush), query head h reading kv head h / (q_heads/kv_heads).
 * num_splits <= 0 picks the split-K factor; workspace must hold
 * kivi_packed_decode_attention_workspace_size(...) bytes (0 means none is
 * needed and workspace may be NULL).  Supported: any q_heads that is a
 * multiple of kv_heads (more than 8 query heads per kv head run one launch
 * per group of 8, each streaming the store once), head_dim % 16 == 0 and
 * <= 256; plain-layout stores also need
 * group_size_k % 16 == 0 and <= 64.  Matrix-core-layout stores run on the
 * bf16 MFMA units with fp32 accumulation (relative error ~1e-5), forming
 * products in units of 2^-64: key scales and key products
 * q*k_scale*softmax_scale*log2(e) must stay below 2^59 and value scales
 * below 2^51 (beyond, the output is inf or NaN); value products below
 * ~2^-38 lose relative precision. */
/* 0 if kivi_packed_decode_attention can run a store of this geometry (for
 * any context length), else the KIVI_ERR_* code its launch would return, with
 * the message in kivi_last_error().  No reference counterpart; it lets a
 * cache refuse a geometry when it is built instead of at its first decode. */
int kivi_packed_decode_attention_supported(int32_t q_heads, int32_t kv_heads,
                                           int32_t head_dim, int32_t group_size_k,
                                           int32_t group_size_v);

size_t kivi_packed_decode_attention_workspace_size(int32_t batch, int32_t q_heads,
                                                   int32_t kv_heads, int32_t head_dim,
                                                   int32_t group_size_k, int32_t group_size_v,
                                                   int32_t num_chunks, int32_t res_len,
                                                   int32_t num_splits);

int kivi_packed_decode_attention(const float* q, const uint8_t* k_codes, const float* k_scale,
                                 const float* k_zero, const uint8_t* v_codes,
                                 const float* v_scale, const float* v_zero, const void* k_res,
                                 const void* v_res, int32_t res_dtype, float* out, void* workspace,
                                 size_t workspace_bytes, int32_t batch, int32_t q_heads,
                                 int32_t kv_heads, int32_t head_dim, int32_t group_size_k,
                                 int32_t group_size_v, int32_t chunk_capacity,
                                 int32_t num_chunks, int32_t res_capacity, int32_t res_start,
                                 int32_t res_len, float softmax_scale, int32_t num_splits,
                                 void* stream);

/* Size of the device-resident scratch array behind
 * kivi_packed_decode_attention_noalloc: 8 MiB per GPU, held until the process
 * ends. */
#define KIVI_NOALLOC_SCRATCH_BYTES (8u << 20)

/* kivi_packed_decode_attention without a workspace argument and without any
 * allocation: no reference counterpart; it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  Same arguments (minus workspace), same
 * kernels and the same result bit for bit.  The split partials live in a
 * library-owned device array of KIVI_NOALLOC_SCRATCH_BYTES per GPU, whose
 * address is resolved on the first call made with that GPU current.  A launch
 * whose partials exceed that size (kivi_packed_decode_attention_workspace_size)
 * is rejected with KIVI_ERR_INVALID_ARGUMENT before anything runs.  Every call
 * on one GPU shares that GPU's array: calls that overlap on one GPU (on
 * different streams, unordered) race and must not be issued. */
int kivi_packed_decode_attention_noalloc(
    const float* q, const uint8_t* k_codes, const float* k_scale, const float* k_zero,
    const uint8_t* v_codes, const float* v_scale, const float* v_zero, const void* k_res,
    const void* v_res, int32_t res_dtype, float* out, int32_t batch, int32_t q_heads,
    int32_t kv_heads, int32_t head_dim, int32_t group_size_k, int32_t group_size_v,
    int32_t chunk_capacity, int32_t num_chunks, int32_t res_capacity, int32_t res_start,
    int32_t res_len, float softmax_scale, int32_t num_splits, void* stream);

/* Attention of q_len query tokens per sequence over the packed store and the
 * residual window: q and out are [batch][q_len][q_heads][head_dim] f32; all
 * other arguments as for kivi_packed_decode_attention (q_len = 1 is that
 * call, and one token always sees the whole context).  causal != 0 with
 * q_len > 1: the query tokens are the window's last q_len tokens (res_len >=
 * q_len) and token i sees every quantised token and the window up to itself
 * -- a forward of q_len tokens on a non-empty cache (chunked prefill,
 * speculative verification), HF's causal mask over [cache ; new tokens].
 * causal == 0: every token sees the whole context (the reference's own
 * q_len = 3 attention check, tests/integration/test_attention_fix.py:19-43).
 * kv_start: NULL, or a device array of batch int32 -- sequence b's first
 * visible context position (a left-padded batch: HF's attention mask hides
 * positions 0 .. kv_start[b]-1, quantised or in the window); each must leave
 * every query token at least one visible position (for causal queries:
 * kv_start[b] <= num_chunks*G + res_len - q_len).
 * When q_len * (q_heads / kv_heads) exceeds 8 the tokens are split over
 * several launches (and more than 8 query heads per kv head into groups of
 * 8), each streaming the store once.  No reference counterpart
 * beyond that math (the reference runs HF attention on the CPU,
 * src/kivi_sycl/cache/manager.py:251-290). */
size_t kivi_packed_attention_workspace_size(int32_t batch, int32_t q_len, int32_t q_heads,
                                            int32_t kv_heads, int32_t head_dim,
                                            int32_t group_size_k, int32_t group_size_v,
                                            int32_t num_chunks, int32_t res_len,
                                            int32_t num_splits);

int kivi_packed_attention(const float* q, int32_t q_len, int32_t causal,
                          const int32_t* kv_start, const uint8_t* k_codes,
                          const float* k_scale, const float* k_zero, const uint8_t* v_codes,
                          const float* v_scale, const float* v_zero, const void* k_res,
                          const void* v_res, int32_t res_dtype, float* out, void* workspace,
                          size_t workspace_bytes, int32_t batch, int32_t q_heads,
                          int32_t kv_heads, int32_t head_dim, int32_t group_size_k,
                          int32_t group_size_v, int32_t chunk_capacity, int32_t num_chunks,
                          int32_t res_capacity, int32_t res_start, int32_t res_len,
                          float softmax_scale, int32_t num_splits, void* stream);

/* kivi_packed_attention with any padding pattern: hidden (NULL: none) holds
 * one row of hidden_stride uint32 words per sequence, bit p % 32 of word
 * p / 32 of row b set when context position p (0 .. num_chunks*G + res_len
 * - 1: the quantised tokens, then the window oldest first) is hidden from
 * every query token of sequence b; hidden_stride >= ceil(context / 32).
 * Positions before kv_start[b] (if given) are hidden as well, and causal
 * queries see the window up to themselves as in kivi_packed_attention.  A
 * query row that sees no position at all (padding rows) gets zeros.  Covers
 * HF attention masks of right-padded batches and batches with holes: a
 * key-padding mask combined with the causal rule (the reference feeds any
 * such mask to HF attention over get_full_cache(),
 * src/kivi_sycl/generation/generate.py:76 and
 * src/kivi_sycl/cache/manager.py:251-290). */
int kivi_packed_attention_masked(const float* q, int32_t q_len, int32_t causal,
                                 const int32_t* kv_start, const uint32_t* hidden,
                                 int64_t hidden_stride, const uint8_t* k_codes,
                                 const float* k_scale, const float* k_zero,
                                 const uint8_t* v_codes, const float* v_scale,
                                 const float* v_zero, const void* k_res, const void* v_res,
                                 int32_t res_dtype, float* out, void* workspace,
                                 size_t workspace_bytes, int32_t batch, int32_t q_heads,
                                 int32_t kv_heads, int32_t head_dim, int32_t group_size_k,
                                 int32_t group_size_v, int32_t chunk_capacity,
                                 int32_t num_chunks, int32_t res_capacity, int32_t res_start,
                                 int32_t res_len, float softmax_scale, int32_t num_splits,
                                 void* stream);

/* kivi_packed_decode_attention with this step's new token appended in the
 * same launch: the window (res_start, res_len) already counts the new token
 * as its last (index res_len - 1, ring slot (res_start + res_len - 1) %
 * res_capacity); the kernel reads it from k_new / v_new (element type
 * res_dtype, element (b, h, d) at b*new_batch_stride + h*new_head_stride + d,
 * rows aligned to four elements: 16 bytes for f32, 8 for bf16/f16) and writes
 * it into that ring slot for later launches.  Same
 * result as kivi_store_append followed by kivi_packed_decode_attention,
 * without the separate launch.  Replaces the residual append of
 * KiviCache.add_tokens (manager.py:226-231) together with the step's
 * attention. */
int kivi_packed_decode_attention_append(
    const float* q, const void* k_new, const void* v_new, int64_t new_batch_stride,
    int64_t new_head_stride, const uint8_t* k_codes, const float* k_scale, const float* k_zero,
    const uint8_t* v_codes, const float* v_scale, const float* v_zero, void* k_res,
    void* v_res, int32_t res_dtype, float* out, void* workspace, size_t workspace_bytes, int32_t batch,
    int32_t q_heads, int32_t kv_heads, int32_t head_dim, int32_t group_size_k,
    int32_t group_size_v, int32_t chunk_capacity, int32_t num_chunks, int32_t res_capacity,
    int32_t res_start, int32_t res_len, float softmax_scale, int32_t num_splits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KIVI_HIP_H */
