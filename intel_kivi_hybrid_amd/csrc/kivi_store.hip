// HBM-resident packed KV store: flush of the oldest residual tokens into 2-bit
// chunks.
//
// Replaces KiviCache._flush_group (src/kivi_sycl/cache/manager.py:309-374):
// instead of transposing on the host, copying to the device, round-tripping,
// copying back and concatenating a CPU history, one kernel reads the G oldest
// tokens of every (batch, kv-head) straight out of the device residual ring and
// writes the packed chunk (and, optionally, the dequantised tokens the served
// cache needs) in place.
//
// Store layout per (b, kv-head), chunk c of G tokens (chunk-major so a flush
// appends one contiguous block and attention streams whole chunks):
//   k_codes [C][G][D/4]   token-major: byte (t, i) holds channels 4i..4i+3 of
//                         token t, channel 4i+k at bits 2k (codes of the
//                         per-channel quantisation along the chunk's tokens)
//   k_scale/k_zero [C][D] one group per channel per chunk
//   v_codes [C][D][G/4]   channel-major: byte (d, j) holds tokens 4j..4j+3 of
//                         channel d, token 4j+k at bits 2k (codes of the
//                         per-token quantisation along channels)
//   v_scale/v_zero [C][G][D/Gv]
// The codes, scales and zeros are those quantize_keys produces on the chunk's
// [D, G] transpose and quantize_values on its [G, D] rows; only the byte order
// of the codes differs (each is the transpose of the reference byte order).
#include "kivi_common.hpp"
#include "../../include/kivi_hip.h"

namespace kivi {
namespace {

constexpr int kFlushBlock = 256;

struct FlushArgs {
    const float* k_res;   // [B, H, Rcap, D]
    const float* v_res;
    uint8_t* k_codes;     // [B, H, Cmax, G, D/4]
    float* k_scale;       // [B, H, Cmax, D]
    float* k_zero;
    uint8_t* v_codes;     // [B, H, Cmax, D, G/4]
    float* v_scale;       // [B, H, Cmax, G, D/Gv]
    float* v_zero;
    float* k_hist;        // optional [B, H, Tcap, D] dequantised keys
    float* v_hist;
    int64_t hist_cap;     // Tcap
    int H, D, G, Gv, Rcap, res_start, Cmax, chunk;
};

// One workgroup per (b, h).  LDS holds the chunk's 2-bit codes as one byte per
// element, [G][D], so the two transposed byte orders can be assembled.
__global__ __launch_bounds__(kFlushBlock) void flush_kernel(FlushArgs a) {
    extern __shared__ uint8_t codes[];           // [G][D]
    const int bh = blockIdx.x;                   // b * H + h
    const int D = a.D, G = a.G, Gv = a.Gv;
    const int64_t res_base = (int64_t)bh * a.Rcap * D;
    const int64_t chunk_id = (int64_t)bh * a.Cmax + a.chunk;
    const int64_t hist_row0 = a.k_hist ? ((int64_t)bh * a.hist_cap + (int64_t)a.chunk * G) : 0;

    // ---- keys: per-channel groups along the chunk's G tokens ----------------
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float mn = 1e30f, mx = -1e30f;
        for (int t = 0; t < G; ++t) {
            int slot = a.res_start + t;
            if (slot >= a.Rcap) slot -= a.Rcap;
            const float x = a.k_res[res_base + (int64_t)slot * D + d];
            mn = fmin_nan(mn, x);
            mx = fmax_nan(mx, x);
        }
        float scale;
        finish_group(mn, mx, scale);
        a.k_scale[chunk_id * D + d] = scale;
        a.k_zero[chunk_id * D + d] = mn;
        for (int t = 0; t < G; ++t) {
            int slot = a.res_start + t;
            if (slot >= a.Rcap) slot -= a.Rcap;
            const float x = a.k_res[res_base + (int64_t)slot * D + d];
            const uint32_t q = code_exact(x, mn, scale);
            codes[t * D + d] = (uint8_t)q;
            if (a.k_hist) a.k_hist[(hist_row0 + t) * D + d] = decode1(q, scale, mn);
        }
    }
    __syncthreads();
    // token-major bytes: (t, i) <- channels 4i..4i+3
    const int kbytes = G * (D / 4);
    for (int e = threadIdx.x; e < kbytes; e += blockDim.x) {
        const int t = e / (D / 4), i = e % (D / 4);
        const uint8_t* c = &codes[t * D + 4 * i];
        a.k_codes[chunk_id * kbytes + e] = (uint8_t)(c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6));
    }
    __syncthreads();

    // ---- values: per-token groups of Gv channels -----------------------------
    const int gpt = D / Gv;
    for (int e = threadIdx.x; e < G * gpt; e += blockDim.x) {
        const int t = e / gpt, gi = e % gpt;
        int slot = a.res_start + t;
        if (slot >= a.Rcap) slot -= a.Rcap;
        const float* x = a.v_res + res_base + (int64_t)slot * D + gi * Gv;
        float mn = 1e30f, mx = -1e30f;
        for (int j = 0; j < Gv; ++j) {
            mn = fmin_nan(mn, x[j]);
            mx = fmax_nan(mx, x[j]);
        }
        float scale;
        finish_group(mn, mx, scale);
        a.v_scale[(chunk_id * G + t) * gpt + gi] = scale;
        a.v_zero[(chunk_id * G + t) * gpt + gi] = mn;
        for (int j = 0; j < Gv; ++j) {
            const uint32_t q = code_exact(x[j], mn, scale);
            codes[t * D + gi * Gv + j] = (uint8_t)q;
            if (a.v_hist) a.v_hist[(hist_row0 + t) * D + gi * Gv + j] = decode1(q, scale, mn);
        }
    }
    __syncthreads();
    // channel-major bytes: (d, j) <- tokens 4j..4j+3
    const int vbytes = D * (G / 4);
    for (int e = threadIdx.x; e < vbytes; e += blockDim.x) {
        const int d = e / (G / 4), j = e % (G / 4);
        const uint8_t c0 = codes[(4 * j) * D + d], c1 = codes[(4 * j + 1) * D + d];
        const uint8_t c2 = codes[(4 * j + 2) * D + d], c3 = codes[(4 * j + 3) * D + d];
        a.v_codes[chunk_id * vbytes + e] = (uint8_t)(c0 | (c1 << 2) | (c2 << 4) | (c3 << 6));
    }
}

}  // namespace
}  // namespace kivi

using namespace kivi;

extern "C" int kivi_store_flush(const float* k_res, const float* v_res, uint8_t* k_codes,
                                float* k_scale, float* k_zero, uint8_t* v_codes,
                                float* v_scale, float* v_zero, float* k_hist, float* v_hist,
                                int64_t hist_capacity, int32_t batch, int32_t kv_heads,
                                int32_t head_dim, int32_t group_size_k,
                                int32_t group_size_v, int32_t res_capacity,
                                int32_t res_start, int32_t chunk_capacity,
                                int32_t chunk_index, void* stream) {
    if (!k_res || !v_res || !k_codes || !k_scale || !k_zero || !v_codes || !v_scale || !v_zero)
        return set_error(kErrInvalidArgument, "null tensor pointer");
    if ((k_hist == nullptr) != (v_hist == nullptr))
        return set_error(kErrInvalidArgument, "k_hist and v_hist must both be given or both null");
    if (batch <= 0 || kv_heads <= 0)
        return set_error(kErrInvalidArgument, "batch and kv_heads must be positive");
    if (head_dim <= 0 || head_dim % 4)
        return set_error(kErrInvalidArgument, "head_dim must be positive and divisible by 4");
    if (group_size_k <= 0 || group_size_k % 4)
        return set_error(kErrInvalidArgument,
                         "group_size must be positive and divisible by 4, got %d", group_size_k);
    if (group_size_v <= 0 || group_size_v % 4 || head_dim % group_size_v)
        return set_error(kErrInvalidArgument,
                         "head_dim must be positive and divisible by group_size");
    if (res_capacity < group_size_k)
        return set_error(kErrInvalidArgument, "residual capacity %d is below group_size %d",
                         res_capacity, group_size_k);
    if (res_start < 0 || res_start >= res_capacity)
        return set_error(kErrInvalidArgument, "res_start %d outside [0, %d)", res_start,
                         res_capacity);
    if (chunk_index < 0 || chunk_index >= chunk_capacity)
        return set_error(kErrInvalidArgument, "chunk %d outside capacity %d", chunk_index,
                         chunk_capacity);
    if (k_hist && (int64_t)(chunk_index + 1) * group_size_k > hist_capacity)
        return set_error(kErrInvalidArgument, "history capacity %lld too small",
                         (long long)hist_capacity);
    const size_t lds = (size_t)group_size_k * head_dim;
    if (lds > 64 * 1024)
        return set_error(kErrUnsupported, "group_size_k * head_dim = %zu exceeds 65536", lds);
    FlushArgs a{k_res, v_res, k_codes, k_scale, k_zero, v_codes, v_scale, v_zero,
                k_hist, v_hist, hist_capacity, kv_heads, head_dim, group_size_k,
                group_size_v, res_capacity, res_start, chunk_capacity, chunk_index};
    flush_kernel<<<batch * kv_heads, kFlushBlock, lds, (hipStream_t)stream>>>(a);
    return check_launch("store_flush");
}
