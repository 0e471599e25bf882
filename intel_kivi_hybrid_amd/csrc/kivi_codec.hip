// KIVI 2-bit asymmetric codec for gfx950: quantise + pack, unpack +
// dequantise, and the fused round-trip.
//
// Replaces the reference's six SYCL kernels
// (src/csrc/kernels/quantize_kernels.cpp:24-120,
//  src/csrc/kernels/dequantize_kernels.cpp:32-124,
//  src/csrc/kernels/roundtrip_kernels.cpp:14-91).  Keys (per channel, grouped
// along tokens) and values (per token, grouped along channels) both reduce
// contiguous runs of G floats and write group g's bytes at g*G/4, so one
// flat-group kernel body serves both.
//
// Layout of the work (wave64): lane i of a wave loads float4 number i of a
// 64-float4 tile, so every load instruction reads 1 KiB contiguously.  A group
// of G floats is G/4 consecutive lanes; its min/max is a segmented butterfly
// (DPP quad permutes and row mirrors, then ds_swizzle / ds_bpermute for 32/64
// lanes).  Each lane turns its 4 floats into one packed byte in registers.
// Group sizes whose G/4 is not a power of two <= 64 take a one-thread-per-
// group kernel with the same arithmetic.
#include <tuple>

#include "kivi_common.hpp"
#include "../../include/kivi_hip.h"

namespace kivi {
namespace {

constexpr int kBlock = 256;
constexpr int kUnroll = 4;
constexpr int kQuantVPL = 2;        // float4s per segment in quantize_vec_kernel
constexpr int kQuantIters = 1;      // segments per thread in quantize_vec_kernel (2 and 4
                                    // measured slower at config 2: 230 and 237 us per pair)

__device__ __forceinline__ void min_max4(const float4& v, float& mn, float& mx) {
    mn = fmin_nan(fmin_nan(v.x, v.y), fmin_nan(v.z, v.w));
    mx = fmax_nan(fmax_nan(v.x, v.y), fmax_nan(v.z, v.w));
}

// ----------------------------------------------------------------------------
// Segmented kernels: LANES = G/4 lanes per group.
// ----------------------------------------------------------------------------
template <int LANES>
__global__ __launch_bounds__(kBlock) void quantize_seg_kernel(
    const float4* __restrict__ in, uint8_t* __restrict__ packed,
    float* __restrict__ scales, float* __restrict__ zeros, int64_t n_vec) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t base = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t idx = base + (int64_t)u * kBlock;
        v[u] = idx < n_vec ? in[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t idx = base + (int64_t)u * kBlock;
        float mn, mx, scale;
        min_max4(v[u], mn, mx);
        seg_min_max<LANES>(mn, mx);
        finish_group(mn, mx, scale);
        const uint32_t byte = encode4(v[u].x, v[u].y, v[u].z, v[u].w, mn, scale);
        if (idx < n_vec) {
            packed[idx] = (uint8_t)byte;
            if ((lane & (LANES - 1)) == 0) {
                scales[idx / LANES] = scale;
                zeros[idx / LANES] = mn;
            }
        }
    }
}

// Segment kernels: a segment is VPL consecutive float4s of a group, LANES =
// G/(4*VPL) adjacent lanes per group.  Larger segments mean fewer cross-lane
// reduction steps and fewer scale divisions per element; each load
// instruction then reads 16 bytes per lane at a VPL*16-byte stride.  A thread
// takes ITERS segments one grid stride apart, all loads issued first, so
// that a wave has more bytes in flight at the same coalescing.
// Outputs use streaming stores, and with VPL == 2 and PAIR (codes 4-byte
// aligned) adjacent lanes combine their two code bytes into one 32-bit
// store: a read-only stream of config 2's shape runs in 89 us per launch,
// with one 16-bit code store per lane and 64-byte scale/zero stores per wave
// in 107 us, with paired codes and streaming stores in 102 us.
template <int LANES, int VPL, int ITERS, bool PAIR>
__global__ __launch_bounds__(kBlock) void quantize_vec_kernel(
    const float4* __restrict__ in, uint8_t* __restrict__ packed,
    float* __restrict__ scales, float* __restrict__ zeros, int64_t n_seg) {
    const int64_t t0 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int64_t stride = (int64_t)gridDim.x * kBlock;   // a multiple of LANES
    // Groups are whole (n_seg % LANES == 0) and a group's lanes share an
    // iteration, so a group is either wholly in range or wholly past it;
    // past-the-end lanes reload the last segment and store nothing.
    float4 v[ITERS][VPL];
#pragma unroll
    for (int u = 0; u < ITERS; ++u) {
        const int64_t t = min(t0 + u * stride, n_seg - 1);
#pragma unroll
        for (int j = 0; j < VPL; ++j) v[u][j] = in[t * VPL + j];
    }
#pragma unroll
    for (int u = 0; u < ITERS; ++u) {
        const int64_t t = t0 + u * stride;
        float mn, mx, scale;
        min_max4(v[u][0], mn, mx);
#pragma unroll
        for (int j = 1; j < VPL; ++j) {
            float a, b;
            min_max4(v[u][j], a, b);
            mn = fmin_nan(mn, a);
            mx = fmax_nan(mx, b);
        }
        seg_min_max<LANES>(mn, mx);
        finish_group(mn, mx, scale);
        uint32_t bytes[VPL];
#pragma unroll
        for (int j = 0; j < VPL; ++j)
            bytes[j] = encode4(v[u][j].x, v[u][j].y, v[u][j].z, v[u][j].w, mn, scale);
        if (t >= n_seg) continue;
        if constexpr (VPL % 4 == 0) {
#pragma unroll
            for (int j = 0; j < VPL; j += 4)
                reinterpret_cast<uint32_t*>(packed + t * VPL)[j / 4] =
                    bytes[j] | (bytes[j + 1] << 8) | (bytes[j + 2] << 16) | (bytes[j + 3] << 24);
        } else if constexpr (VPL == 2) {
            const uint32_t mine = bytes[0] | (bytes[1] << 8);
            if constexpr (PAIR) {
                // lanes 2k, 2k+1 hold segments t, t+1 (never split by the end:
                // n_seg is a whole number of groups of LANES >= 2 lanes)
                const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(
                    0, (int)mine, 0xB1, 0xF, 0xF, false);     // quad_perm [1,0,3,2]
                if ((threadIdx.x & 1) == 0)
                    store_stream(reinterpret_cast<uint32_t*>(packed) + t / 2, mine | (other << 16));
            } else {
                reinterpret_cast<uint16_t*>(packed)[t] = (uint16_t)mine;
            }
        } else {
#pragma unroll
            for (int j = 0; j < VPL; ++j) packed[t * VPL + j] = (uint8_t)bytes[j];
        }
        if ((threadIdx.x & (LANES - 1)) == 0) {
            store_stream(scales + t / LANES, scale);
            store_stream(zeros + t / LANES, mn);
        }
    }
}

template <int LANES>
__global__ __launch_bounds__(kBlock) void roundtrip_seg_kernel(
    const float4* __restrict__ in, float4* __restrict__ out, int64_t n_vec) {
    const int64_t base = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    float4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t idx = base + (int64_t)u * kBlock;
        v[u] = idx < n_vec ? in[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t idx = base + (int64_t)u * kBlock;
        float mn, mx, scale;
        min_max4(v[u], mn, mx);
        seg_min_max<LANES>(mn, mx);
        finish_group(mn, mx, scale);
        const uint32_t byte = encode4(v[u].x, v[u].y, v[u].z, v[u].w, mn, scale);
        if (idx < n_vec) store_stream(out + idx, decode4(byte, scale, mn));
    }
}

// ----------------------------------------------------------------------------
// One thread per group: any G divisible by 4, any alignment.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void serial_group_stats(const float* x, int G, float& mn,
                                                   float& mx, float& scale) {
    mn = 1e30f;
    mx = -1e30f;
    for (int i = 0; i < G; i += 4) {
        float lmn = fmin_nan(fmin_nan(x[i], x[i + 1]), fmin_nan(x[i + 2], x[i + 3]));
        float lmx = fmax_nan(fmax_nan(x[i], x[i + 1]), fmax_nan(x[i + 2], x[i + 3]));
        mn = fmin_nan(mn, lmn);
        mx = fmax_nan(mx, lmx);
    }
    finish_group(mn, mx, scale);
}

__global__ __launch_bounds__(kBlock) void quantize_serial_kernel(
    const float* __restrict__ in, uint8_t* __restrict__ packed,
    float* __restrict__ scales, float* __restrict__ zeros, int64_t n_groups, int G) {
    const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (g >= n_groups) return;
    const float* x = in + g * G;
    float mn, mx, scale;
    serial_group_stats(x, G, mn, mx, scale);
    scales[g] = scale;
    zeros[g] = mn;
    uint8_t* o = packed + g * (G / 4);
    for (int j = 0; j < G / 4; ++j)
        o[j] = (uint8_t)encode4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3], mn, scale);
}

__global__ __launch_bounds__(kBlock) void roundtrip_serial_kernel(
    const float* __restrict__ in, float* __restrict__ out, int64_t n_groups, int G) {
    const int64_t g = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (g >= n_groups) return;
    const float* x = in + g * G;
    float* o = out + g * G;
    float mn, mx, scale;
    serial_group_stats(x, G, mn, mx, scale);
    for (int j = 0; j < G / 4; ++j) {
        const uint32_t b = encode4(x[4 * j], x[4 * j + 1], x[4 * j + 2], x[4 * j + 3], mn, scale);
        const float4 d = decode4(b, scale, mn);
        o[4 * j] = d.x;
        o[4 * j + 1] = d.y;
        o[4 * j + 2] = d.z;
        o[4 * j + 3] = d.w;
    }
}

// ----------------------------------------------------------------------------
// Dequantise: one lane per packed byte -> one float4 (lane-contiguous 16 B
// stores, so each store instruction writes 1 KiB).  BPG = G/4 bytes per group
// when it is a power of two (shift), 0 for the generic divide.
// ----------------------------------------------------------------------------
template <int BPG, bool kAligned>
__global__ __launch_bounds__(kBlock) void dequantize_kernel(
    const uint8_t* __restrict__ packed, const float* __restrict__ scales,
    const float* __restrict__ zeros, float* __restrict__ out, int64_t n_bytes, int bpg) {
    const int64_t base = (int64_t)blockIdx.x * (kBlock * kUnroll) + threadIdx.x;
    uint32_t b[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t idx = base + (int64_t)u * kBlock;
        b[u] = idx < n_bytes ? (uint32_t)packed[idx] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int64_t idx = base + (int64_t)u * kBlock;
        if (idx >= n_bytes) continue;
        const int64_t g = BPG ? (idx / BPG) : (idx / bpg);
        const float4 d = decode4(b[u], scales[g], zeros[g]);
        if constexpr (kAligned) {
            store_stream(reinterpret_cast<float4*>(out) + idx, d);
        } else {
            store_stream(out + 4 * idx, d.x);
            store_stream(out + 4 * idx + 1, d.y);
            store_stream(out + 4 * idx + 2, d.z);
            store_stream(out + 4 * idx + 3, d.w);
        }
    }
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

inline unsigned grid_for(int64_t items, int64_t per_block) {
    return (unsigned)((items + per_block - 1) / per_block);
}

int check_common(const void* a, const void* b, int64_t n_groups, int32_t G) {
    if (a == nullptr || b == nullptr)
        return set_error(kErrInvalidArgument, "null tensor pointer");
    if (G <= 0 || G % 4 != 0)
        return set_error(kErrInvalidArgument,
                         "group_size must be positive and divisible by 4, got %d", G);
    if (n_groups <= 0)
        return set_error(kErrInvalidArgument, "number of groups must be positive, got %lld",
                         (long long)n_groups);
    if (n_groups > (int64_t(1) << 40) / G)
        return set_error(kErrInvalidArgument, "tensor too large");
    return kOk;
}

}  // namespace

// ----------------------------------------------------------------------------
// Launchers.
// ----------------------------------------------------------------------------
// One kernel launch of kBlock threads per block on `stream`.  With `stop`
// non-null it goes through hipExtLaunchKernel with `stop` as the launch's
// completion event: the event is then signalled by the kernel's own
// dispatch, with no marker packet queued after it (a hipEventRecord marker
// cost ~3.3 us of GPU time between two back-to-back kernels).  Returns the
// extended launch's error; the <<<>>> form's is left for check_launch.
template <class... P, class... A>
int launch(void (*kernel)(P...), unsigned grid, hipStream_t stream, hipEvent_t stop,
           A... args) {
    if (stop == nullptr) {
        kernel<<<grid, kBlock, 0, stream>>>(static_cast<P>(args)...);
        return kOk;
    }
    std::tuple<P...> vals{static_cast<P>(args)...};
    void* ptrs[sizeof...(P)];
    std::apply([&](auto&... v) {
        int i = 0;
        ((ptrs[i++] = static_cast<void*>(&v)), ...);
    }, vals);
    return check_hip(hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), dim3(grid),
                                        dim3(kBlock), ptrs, 0, stream, nullptr, stop, 0),
                     "hipExtLaunchKernel");
}

int launch_quantize_groups(const float* in, uint8_t* packed, float* scales, float* zeros,
                           int64_t n_groups, int32_t G, hipStream_t stream,
                           hipEvent_t stop = nullptr) {
    int rc = check_common(in, packed, n_groups, G);
    if (rc) return rc;
    if (scales == nullptr || zeros == nullptr)
        return set_error(kErrInvalidArgument, "null scales/zeros pointer");
    const int lanes = G / 4;
    const int64_t n_vec = n_groups * lanes;
    const bool pow2 = (lanes & (lanes - 1)) == 0 && lanes <= kWave;
    if (pow2 && aligned16(in) && lanes >= kQuantVPL && kQuantVPL > 1 &&
        ((uintptr_t)packed % (kQuantVPL >= 4 ? 4 : kQuantVPL)) == 0) {
        const int64_t n_seg = n_vec / kQuantVPL;
        const unsigned grid = grid_for(n_seg, kBlock * kQuantIters);
        const float4* in4 = reinterpret_cast<const float4*>(in);
        const bool pair = kQuantVPL == 2 && lanes / kQuantVPL >= 2 && ((uintptr_t)packed % 4) == 0;
        switch (lanes / kQuantVPL) {
#define KIVI_QV(L) case L: \
        if (pair) rc = launch(quantize_vec_kernel<L, kQuantVPL, kQuantIters, true>, grid, stream, stop, in4, packed, scales, zeros, n_seg); \
        else rc = launch(quantize_vec_kernel<L, kQuantVPL, kQuantIters, false>, grid, stream, stop, in4, packed, scales, zeros, n_seg); \
        break;
            KIVI_QV(1) KIVI_QV(2) KIVI_QV(4) KIVI_QV(8) KIVI_QV(16) KIVI_QV(32) KIVI_QV(64)
#undef KIVI_QV
        }
    } else if (pow2 && aligned16(in)) {
        const unsigned grid = grid_for(n_vec, kBlock * kUnroll);
        const float4* in4 = reinterpret_cast<const float4*>(in);
        switch (lanes) {
#define KIVI_Q(L) case L: rc = launch(quantize_seg_kernel<L>, grid, stream, stop, in4, packed, scales, zeros, n_vec); break;
            KIVI_Q(1) KIVI_Q(2) KIVI_Q(4) KIVI_Q(8) KIVI_Q(16) KIVI_Q(32) KIVI_Q(64)
#undef KIVI_Q
        }
    } else {
        rc = launch(quantize_serial_kernel, grid_for(n_groups, kBlock), stream, stop, in, packed, scales, zeros, n_groups, G);
    }
    if (rc) return rc;
    return check_launch("quantize");
}

int launch_roundtrip_groups(const float* in, float* out, int64_t n_groups, int32_t G,
                            hipStream_t stream, hipEvent_t stop = nullptr) {
    int rc = check_common(in, out, n_groups, G);
    if (rc) return rc;
    const int lanes = G / 4;
    const int64_t n_vec = n_groups * lanes;
    const bool pow2 = (lanes & (lanes - 1)) == 0 && lanes <= kWave;
    if (pow2 && aligned16(in) && aligned16(out)) {
        const unsigned grid = grid_for(n_vec, kBlock * kUnroll);
        const float4* in4 = reinterpret_cast<const float4*>(in);
        float4* out4 = reinterpret_cast<float4*>(out);
        switch (lanes) {
#define KIVI_R(L) case L: rc = launch(roundtrip_seg_kernel<L>, grid, stream, stop, in4, out4, n_vec); break;
            KIVI_R(1) KIVI_R(2) KIVI_R(4) KIVI_R(8) KIVI_R(16) KIVI_R(32) KIVI_R(64)
#undef KIVI_R
        }
    } else {
        rc = launch(roundtrip_serial_kernel, grid_for(n_groups, kBlock), stream, stop, in, out, n_groups, G);
    }
    if (rc) return rc;
    return check_launch("quant_dequant_roundtrip");
}

int launch_dequantize_groups(const uint8_t* packed, const float* scales, const float* zeros,
                             float* out, int64_t n_groups, int32_t G, hipStream_t stream,
                             hipEvent_t stop = nullptr) {
    int rc = check_common(packed, out, n_groups, G);
    if (rc) return rc;
    if (scales == nullptr || zeros == nullptr)
        return set_error(kErrInvalidArgument, "null scales/zeros pointer");
    const int bpg = G / 4;
    const int64_t n_bytes = n_groups * bpg;
    const unsigned grid = grid_for(n_bytes, kBlock * kUnroll);
    const bool al = aligned16(out);
    switch (bpg) {
#define KIVI_D(L) case L: \
        if (al) rc = launch(dequantize_kernel<L, true>, grid, stream, stop, packed, scales, zeros, out, n_bytes, bpg); \
        else rc = launch(dequantize_kernel<L, false>, grid, stream, stop, packed, scales, zeros, out, n_bytes, bpg); \
        break;
        KIVI_D(1) KIVI_D(2) KIVI_D(4) KIVI_D(8) KIVI_D(16) KIVI_D(32) KIVI_D(64)
#undef KIVI_D
        default:
            if (al) rc = launch(dequantize_kernel<0, true>, grid, stream, stop, packed, scales, zeros, out, n_bytes, bpg);
            else rc = launch(dequantize_kernel<0, false>, grid, stream, stop, packed, scales, zeros, out, n_bytes, bpg);
    }
    if (rc) return rc;
    return check_launch("dequantize");
}

}  // namespace kivi

using namespace kivi;

static int check_values(int64_t num_tokens, int32_t head_dim, int32_t G) {
    if (G <= 0 || G % 4 != 0)
        return set_error(kErrInvalidArgument,
                         "group_size must be positive and divisible by 4, got %d", G);
    if (head_dim <= 0 || head_dim % G != 0)
        return set_error(kErrInvalidArgument,
                         "head_dim must be positive and divisible by group_size");
    if (num_tokens <= 0)
        return set_error(kErrInvalidArgument, "input must be non-empty");
    return kOk;
}

extern "C" {

int kivi_quantize_keys_per_channel(const float* input, uint8_t* output, float* scales,
                                   float* zeros, int64_t num_channels, int32_t group_size,
                                   void* stream) {
    return launch_quantize_groups(input, output, scales, zeros, num_channels, group_size,
                                  (hipStream_t)stream);
}

int kivi_quantize_values_per_token(const float* input, uint8_t* output, float* scales,
                                   float* zeros, int64_t num_tokens, int32_t head_dim,
                                   int32_t group_size, void* stream) {
    int rc = check_values(num_tokens, head_dim, group_size);
    if (rc) return rc;
    return launch_quantize_groups(input, output, scales, zeros,
                                  num_tokens * (head_dim / group_size), group_size,
                                  (hipStream_t)stream);
}

int kivi_dequantize_keys_per_channel(const uint8_t* input, const float* scales,
                                     const float* zeros, float* output, int64_t num_channels,
                                     int32_t group_size, void* stream) {
    return launch_dequantize_groups(input, scales, zeros, output, num_channels, group_size,
                                    (hipStream_t)stream);
}

int kivi_dequantize_values_per_token(const uint8_t* input, const float* scales,
                                     const float* zeros, float* output, int64_t num_groups,
                                     int32_t group_size, void* stream) {
    return launch_dequantize_groups(input, scales, zeros, output, num_groups, group_size,
                                    (hipStream_t)stream);
}

int kivi_quant_dequant_roundtrip_keys(const float* input, float* output,
                                      int64_t num_channels, int32_t group_size,
                                      void* stream) {
    return launch_roundtrip_groups(input, output, num_channels, group_size,
                                   (hipStream_t)stream);
}

int kivi_quant_dequant_roundtrip_values(const float* input, float* output,
                                        int64_t num_tokens, int32_t head_dim,
                                        int32_t group_size, void* stream) {
    int rc = check_values(num_tokens, head_dim, group_size);
    if (rc) return rc;
    return launch_roundtrip_groups(input, output, num_tokens * (head_dim / group_size),
                                   group_size, (hipStream_t)stream);
}

}  // extern "C"

// A new event (timing disabled) handed to `fn` as the stop event of the op's
// kernel launch, and to the caller through *event_out on success.
template <class F>
static int with_stop_event(void** event_out, F&& fn) {
    if (event_out == nullptr)
        return set_error(kErrInvalidArgument, "event_out must not be null");
    *event_out = nullptr;
    hipEvent_t ev = nullptr;
    int rc = check_hip(hipEventCreateWithFlags(&ev, hipEventDisableTiming),
                       "hipEventCreateWithFlags");
    if (rc) return rc;
    rc = fn(ev);
    if (rc) {
        (void)hipEventDestroy(ev);
        return rc;
    }
    *event_out = (void*)ev;
    return kOk;
}

extern "C" {

int kivi_quantize_keys_per_channel_ev(const float* input, uint8_t* output, float* scales,
                                      float* zeros, int64_t num_channels, int32_t group_size,
                                      void* stream, void** event_out) {
    return with_stop_event(event_out, [&](hipEvent_t ev) {
        return launch_quantize_groups(input, output, scales, zeros, num_channels, group_size,
                                      (hipStream_t)stream, ev);
    });
}

int kivi_quantize_values_per_token_ev(const float* input, uint8_t* output, float* scales,
                                      float* zeros, int64_t num_tokens, int32_t head_dim,
                                      int32_t group_size, void* stream, void** event_out) {
    if (event_out) *event_out = nullptr;
    int rc = check_values(num_tokens, head_dim, group_size);
    if (rc) return rc;
    return with_stop_event(event_out, [&](hipEvent_t ev) {
        return launch_quantize_groups(input, output, scales, zeros,
                                      num_tokens * (head_dim / group_size), group_size,
                                      (hipStream_t)stream, ev);
    });
}

int kivi_dequantize_keys_per_channel_ev(const uint8_t* input, const float* scales,
                                        const float* zeros, float* output,
                                        int64_t num_channels, int32_t group_size, void* stream,
                                        void** event_out) {
    return with_stop_event(event_out, [&](hipEvent_t ev) {
        return launch_dequantize_groups(input, scales, zeros, output, num_channels, group_size,
                                        (hipStream_t)stream, ev);
    });
}

int kivi_dequantize_values_per_token_ev(const uint8_t* input, const float* scales,
                                        const float* zeros, float* output, int64_t num_groups,
                                        int32_t group_size, void* stream, void** event_out) {
    return with_stop_event(event_out, [&](hipEvent_t ev) {
        return launch_dequantize_groups(input, scales, zeros, output, num_groups, group_size,
                                        (hipStream_t)stream, ev);
    });
}

int kivi_quant_dequant_roundtrip_keys_ev(const float* input, float* output,
                                         int64_t num_channels, int32_t group_size,
                                         void* stream, void** event_out) {
    return with_stop_event(event_out, [&](hipEvent_t ev) {
        return launch_roundtrip_groups(input, output, num_channels, group_size,
                                       (hipStream_t)stream, ev);
    });
}

int kivi_quant_dequant_roundtrip_values_ev(const float* input, float* output,
                                           int64_t num_tokens, int32_t head_dim,
                                           int32_t group_size, void* stream,
                                           void** event_out) {
    if (event_out) *event_out = nullptr;
    int rc = check_values(num_tokens, head_dim, group_size);
    if (rc) return rc;
    return with_stop_event(event_out, [&](hipEvent_t ev) {
        return launch_roundtrip_groups(input, output, num_tokens * (head_dim / group_size),
                                       group_size, (hipStream_t)stream, ev);
    });
}

}  // extern "C"
