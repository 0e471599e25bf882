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
// Per (b, kv-head), chunk c of G tokens holds (layouts in kivi_common.hpp):
//   key codes   : per-channel quantisation along the chunk's G tokens -- the
//                 codes quantize_keys produces on the chunk's [D, G] transpose
//   k_scale/k_zero [D]
//   value codes : per-token quantisation along groups of Gv channels -- the
//                 codes quantize_values produces on the chunk's [G, D] rows
//   v_scale/v_zero [D/Gv][G]
// The codes are byte-for-byte those of the reference ops, only arranged in the
// store's own order (plain or MFMA-operand order).
#include "kivi_common.hpp"
#include "../../include/kivi_hip.h"

namespace kivi {
namespace {

constexpr int kFlushBlock = 256;
constexpr int kTileMaxElems = 8192;   // G*D staged in LDS (fp32 tile + u8 codes)

struct FlushArgs {
    const float* k_res;   // [B, H, Rcap, D]
    const float* v_res;
    uint8_t* k_codes;     // [B, H, Cmax, G*D/4]
    float* k_scale;       // [B, H, Cmax, D]
    float* k_zero;
    uint8_t* v_codes;     // [B, H, Cmax, G*D/4]
    float* v_scale;       // [B, H, Cmax, D/Gv, G]
    float* v_zero;
    float* k_hist;        // optional [B, H, Tcap, D] dequantised keys
    float* v_hist;
    int64_t hist_cap;     // Tcap
    int D, G, Gv, Rcap, res_start, Cmax, chunk;
};

__device__ __forceinline__ int ring(int start, int t, int cap) {
    const int s = start + t;
    return s >= cap ? s - cap : s;
}

// Writes one chunk's codes (u8 per element in `codes`, [G][D]) in the store
// layout.  KEY selects the key (token-block x channel-step) or value
// (token-step x channel-block) tiling of the MFMA layout.
template <int LAYOUT, bool KEY>
__device__ void write_codes(const uint8_t* codes, uint8_t* out, int G, int D) {
    if constexpr (LAYOUT == kLayoutPlain) {
        if constexpr (KEY) {
            const int n = G * (D / 4);             // byte (t, i): channels 4i..4i+3
            for (int e = threadIdx.x; e < n; e += blockDim.x) {
                const int t = e / (D / 4), i = e % (D / 4);
                const uint8_t* c = codes + t * D + 4 * i;
                out[e] = (uint8_t)(c[0] | (c[1] << 2) | (c[2] << 4) | (c[3] << 6));
            }
        } else {
            const int n = D * (G / 4);             // byte (d, j): tokens 4j..4j+3
            for (int e = threadIdx.x; e < n; e += blockDim.x) {
                const int d = e / (G / 4), j = e % (G / 4);
                out[e] = (uint8_t)(codes[(4 * j) * D + d] | (codes[(4 * j + 1) * D + d] << 2) |
                                   (codes[(4 * j + 2) * D + d] << 4) |
                                   (codes[(4 * j + 3) * D + d] << 6));
            }
        }
    } else {
        const int np = G * D / 1024;               // dwords per lane
        uint32_t* out32 = reinterpret_cast<uint32_t*>(out);
        for (int e = threadIdx.x; e < 64 * np; e += blockDim.x) {
            const int l = e / np, w = e % np;
            uint32_t word = 0;
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const int tile = 2 * w + m;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int t, d;
                    if constexpr (KEY) {
                        const int ks = tile / (G / 16), nb = tile % (G / 16);
                        t = 16 * nb + l % 16;
                        d = 32 * ks + 8 * (l / 16) + j;
                    } else {
                        const int kt = tile / (D / 16), nb = tile % (D / 16);
                        t = 32 * kt + 8 * (l / 16) + j;
                        d = 16 * nb + l % 16;
                    }
                    word |= (uint32_t)codes[t * D + d] << mfma_code_bit(m, j);
                }
            }
            out32[e] = word;
        }
    }
}

// One workgroup per (b, kv-head).  TILE: the chunk's G x D fp32 tokens are
// first staged in LDS with coalesced loads (needs G*D <= kTileMaxElems);
// otherwise elements are read from the residual ring directly.
template <int LAYOUT, bool TILE>
__global__ __launch_bounds__(kFlushBlock) void flush_kernel(FlushArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int D = a.D, G = a.G, Gv = a.Gv, NG = D / Gv;
    float* tile = reinterpret_cast<float*>(smem);                       // [G][D] if TILE
    uint8_t* codes = smem + (TILE ? (size_t)G * D * sizeof(float) : 0); // [G][D]
    const int bh = blockIdx.x;
    const int64_t res_base = (int64_t)bh * a.Rcap * D;
    const int64_t chunk_id = (int64_t)bh * a.Cmax + a.chunk;
    const int64_t code_bytes = (int64_t)G * D / 4;
    const int64_t hist_row0 = (int64_t)bh * a.hist_cap + (int64_t)a.chunk * G;

    auto stage = [&](const float* src) {
        const int nv = G * (D / 4);
        for (int e = threadIdx.x; e < nv; e += blockDim.x) {
            const int t = e / (D / 4), d4 = e % (D / 4);
            const float4 x = reinterpret_cast<const float4*>(
                src + res_base + (int64_t)ring(a.res_start, t, a.Rcap) * D)[d4];
            reinterpret_cast<float4*>(tile)[e] = x;
        }
    };
    auto elem = [&](const float* src, int t, int d) -> float {
        if constexpr (TILE) return tile[t * D + d];
        return src[res_base + (int64_t)ring(a.res_start, t, a.Rcap) * D + d];
    };
    // Dequantised tokens go back into the tile (TILE) and are then copied to
    // the history with coalesced stores.
    auto write_hist = [&](float* hist) {
        if (!hist) return;
        const int nv = G * (D / 4);
        for (int e = threadIdx.x; e < nv; e += blockDim.x) {
            const int t = e / (D / 4), d4 = e % (D / 4);
            reinterpret_cast<float4*>(hist + (hist_row0 + t) * D)[d4] =
                reinterpret_cast<const float4*>(tile)[e];
        }
    };

    // ---- keys: one group per channel, along the chunk's G tokens ----------
    if constexpr (TILE) {
        stage(a.k_res);
        __syncthreads();
    }
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float mn = 1e30f, mx = -1e30f;
        for (int t = 0; t < G; ++t) {
            const float x = elem(a.k_res, t, d);
            mn = fmin_nan(mn, x);
            mx = fmax_nan(mx, x);
        }
        float scale;
        finish_group(mn, mx, scale);
        a.k_scale[chunk_id * D + d] = scale;
        a.k_zero[chunk_id * D + d] = mn;
        for (int t = 0; t < G; ++t) {
            const uint32_t q = code_exact(elem(a.k_res, t, d), mn, scale);
            codes[t * D + d] = (uint8_t)q;
            const float xh = decode1(q, scale, mn);
            if constexpr (TILE) {
                tile[t * D + d] = xh;
            } else if (a.k_hist) {
                a.k_hist[(hist_row0 + t) * D + d] = xh;
            }
        }
    }
    __syncthreads();
    if constexpr (TILE) write_hist(a.k_hist);
    write_codes<LAYOUT, true>(codes, a.k_codes + chunk_id * code_bytes, G, D);
    __syncthreads();

    // ---- values: groups of Gv channels within each token --------------------
    if constexpr (TILE) {
        stage(a.v_res);
        __syncthreads();
    }
    for (int e = threadIdx.x; e < G * NG; e += blockDim.x) {
        const int t = e / NG, gi = e % NG;
        // Start each thread's walk at a different channel so that the LDS
        // reads of neighbouring threads fall in different banks (min/max are
        // order-independent).
        const int rot = threadIdx.x % Gv;
        float mn = 1e30f, mx = -1e30f;
        for (int jj = 0; jj < Gv; ++jj) {
            int j = jj + rot;
            j = j >= Gv ? j - Gv : j;
            const float x = elem(a.v_res, t, gi * Gv + j);
            mn = fmin_nan(mn, x);
            mx = fmax_nan(mx, x);
        }
        float scale;
        finish_group(mn, mx, scale);
        a.v_scale[(chunk_id * NG + gi) * G + t] = scale;
        a.v_zero[(chunk_id * NG + gi) * G + t] = mn;
        for (int jj = 0; jj < Gv; ++jj) {
            int j = jj + rot;
            j = j >= Gv ? j - Gv : j;
            const int d = gi * Gv + j;
            const uint32_t q = code_exact(elem(a.v_res, t, d), mn, scale);
            codes[t * D + d] = (uint8_t)q;
            const float xh = decode1(q, scale, mn);
            if constexpr (TILE) {
                tile[t * D + d] = xh;
            } else if (a.v_hist) {
                a.v_hist[(hist_row0 + t) * D + d] = xh;
            }
        }
    }
    __syncthreads();
    if constexpr (TILE) write_hist(a.v_hist);
    write_codes<LAYOUT, false>(codes, a.v_codes + chunk_id * code_bytes, G, D);
}

}  // namespace
}  // namespace kivi

using namespace kivi;

extern "C" int kivi_store_code_layout(int32_t head_dim, int32_t group_size_k,
                                      int32_t group_size_v) {
    return code_layout_for(head_dim, group_size_k, group_size_v);
}

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
    const int64_t elems = (int64_t)group_size_k * head_dim;
    if (elems > 64 * 1024)
        return set_error(kErrUnsupported, "group_size_k * head_dim = %lld exceeds 65536",
                         (long long)elems);
    const bool aligned = ((uintptr_t)k_res % 16 == 0) && ((uintptr_t)v_res % 16 == 0) &&
                         (!k_hist || ((uintptr_t)k_hist % 16 == 0 && (uintptr_t)v_hist % 16 == 0));
    const bool tile = elems <= kTileMaxElems && aligned;
    const int layout = code_layout_for(head_dim, group_size_k, group_size_v);
    const size_t lds = (size_t)elems * (tile ? sizeof(float) + 1 : 1);
    FlushArgs a{k_res, v_res, k_codes, k_scale, k_zero, v_codes, v_scale, v_zero,
                k_hist, v_hist, hist_capacity, head_dim, group_size_k, group_size_v,
                res_capacity, res_start, chunk_capacity, chunk_index};
    const dim3 grid(batch * kv_heads);
    hipStream_t st = (hipStream_t)stream;
    if (layout == kLayoutMfma) {
        if (tile) flush_kernel<kLayoutMfma, true><<<grid, kFlushBlock, lds, st>>>(a);
        else flush_kernel<kLayoutMfma, false><<<grid, kFlushBlock, lds, st>>>(a);
    } else {
        if (tile) flush_kernel<kLayoutPlain, true><<<grid, kFlushBlock, lds, st>>>(a);
        else flush_kernel<kLayoutPlain, false><<<grid, kFlushBlock, lds, st>>>(a);
    }
    return check_launch("store_flush");
}
