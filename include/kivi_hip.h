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

#define KIVI_HIP_ABI_VERSION 1

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

#ifdef __cplusplus
}
#endif

#endif /* KIVI_HIP_H */
