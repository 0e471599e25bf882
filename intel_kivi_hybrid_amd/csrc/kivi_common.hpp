// Shared host/device helpers for the gfx950 KIVI kernels.
//
// Numerics contract (reference: src/csrc/kernels/internal/quant_tile.hpp:35-91,
// src/csrc/kernels/quantize_kernels.cpp:46-48,
// src/csrc/kernels/dequantize_kernels.cpp:17-28), read as IEEE fp32:
//   min/max over a group, NaN ignored, -0.0 ordered below +0.0, folded with the
//   reference's initial values 1e30f / -1e30f;
//   scale = (max - min) / 3.0f + 1e-10f (correctly rounded divide), zero = min;
//   code  = clamp(round_half_away((x - min) / scale), 0, 3), NaN -> 0;
//   x_hat = fl(fl(code * scale) + zero) (never fused into an FMA).
// The whole library is compiled with -ffp-contract=off and
// -fhip-fp32-correctly-rounded-divide-sqrt; kernels that want FMAs call fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kivi {

constexpr int kWave = 64;

// Clang vector types for nontemporal loads and stores of 16 and 8 bytes.
typedef float kivi_f4v __attribute__((ext_vector_type(4)));
typedef unsigned int kivi_u2v __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Host-side status plumbing (defined in kivi_runtime.hip).
// ---------------------------------------------------------------------------
enum Status : int {
    kOk = 0,
    kErrInvalidArgument = 1,
    kErrLaunch = 2,
    kErrRuntime = 3,
    kErrUnsupported = 4,
};

int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
int check_hip(hipError_t err, const char* what);

// ---------------------------------------------------------------------------
// Packed-store code layouts (shared by the flush and attention kernels).
//
// kLayoutPlain: per chunk of G tokens, key codes [G][D/4] bytes (byte (t, i)
//   holds channels 4i..4i+3 of token t, channel 4i+k at bits 2k) and value
//   codes [D][G/4] bytes (byte (d, j) holds tokens 4j..4j+3 of channel d).
// kLayoutMfma: the chunk's codes are the B operands of
//   v_mfma_f32_16x16x32_bf16, stored lane-major: [64 lanes][NP dwords] per
//   chunk for keys and for values, NP = G*D/1024.  A "tile" is one MFMA B
//   operand: 64 lanes x 8 codes.  Tiles are numbered
//     keys:   tile = ks*(G/16) + nb   (nb: 16-token block, ks: 32-channel step)
//             lane l, element j -> token 16*nb + l%16, channel 32*ks + 8*(l/16) + j
//     values: tile = kt*(D/16) + nb  (kt: 32-token step, nb: 16-channel block)
//             lane l, element j -> token 32*kt + 8*(l/16) + j, channel 16*nb + l%16
//   and tiles 2w and 2w+1 share dword w of each lane: element j of tile
//   2w+m sits at bits  8*m + 2*(j/2) + 16*(j%2).
// Scales/zeros are the same in both layouts: keys [D] per chunk, values
// [D/Gv][G] per chunk (group-major).
// ---------------------------------------------------------------------------
enum CodeLayout : int { kLayoutPlain = 0, kLayoutMfma = 1 };

inline int code_layout_for(int D, int G, int Gv) {
    const bool d_ok = D == 64 || D == 128 || D == 256;
    const bool g_ok = G == 32 || G == 64;
    const bool gv_ok = Gv > 0 && Gv % 32 == 0 && D % Gv == 0;
    return (d_ok && g_ok && gv_ok) ? kLayoutMfma : kLayoutPlain;
}

__host__ __device__ constexpr int mfma_code_bit(int m, int j) {
    return 8 * m + 2 * (j / 2) + 16 * (j % 2);
}

// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------

// fmin/fmax with NaN ignored.  v_min_f32 / v_max_f32 order -0.0 below +0.0.
__device__ __forceinline__ float fmin_nan(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ float fmax_nan(float a, float b) { return fmaxf(a, b); }

// Cross-lane exchange helpers within a wave64.  `seg_partner<M>` returns the value
// held by lane (lane ^ M).  Masks 1 and 2 use DPP quad permutes, 4 and 8 use
// the row half-mirror / mirror (valid for reductions once the smaller
// sub-segments already hold their reduced value), 16 and 32 use ds_swizzle /
// ds_bpermute.
template <int M>
__device__ __forceinline__ float seg_partner(float v) {
    int x = __builtin_bit_cast(int, v);
    int r;
    if constexpr (M == 1) {
        r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);   // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);   // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);  // row_half_mirror
    } else if constexpr (M == 8) {
        r = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);  // row_mirror
    } else if constexpr (M == 16) {
        r = __builtin_amdgcn_ds_swizzle(x, 0x401F);                      // bitmask xor 0x10
    } else {
        static_assert(M == 32, "segment partner mask");
        r = __shfl_xor(x, 32);
    }
    return __builtin_bit_cast(float, r);
}

// Reduce min and max over aligned segments of LANES consecutive lanes
// (LANES a power of two <= 64).  Every lane of a segment ends with the result.
template <int LANES>
__device__ __forceinline__ void seg_min_max(float& mn, float& mx) {
    if constexpr (LANES >= 2) {
        mn = fmin_nan(mn, seg_partner<1>(mn));
        mx = fmax_nan(mx, seg_partner<1>(mx));
    }
    if constexpr (LANES >= 4) {
        mn = fmin_nan(mn, seg_partner<2>(mn));
        mx = fmax_nan(mx, seg_partner<2>(mx));
    }
    if constexpr (LANES >= 8) {
        mn = fmin_nan(mn, seg_partner<4>(mn));
        mx = fmax_nan(mx, seg_partner<4>(mx));
    }
    if constexpr (LANES >= 16) {
        mn = fmin_nan(mn, seg_partner<8>(mn));
        mx = fmax_nan(mx, seg_partner<8>(mx));
    }
    if constexpr (LANES >= 32) {
        mn = fmin_nan(mn, seg_partner<16>(mn));
        mx = fmax_nan(mx, seg_partner<16>(mx));
    }
    if constexpr (LANES >= 64) {
        mn = fmin_nan(mn, seg_partner<32>(mn));
        mx = fmax_nan(mx, seg_partner<32>(mx));
    }
}

// Fold the reference's initial values (quant_tile.hpp:39-40) and form the
// group's scale (quantize_kernels.cpp:46).
__device__ __forceinline__ void finish_group(float& mn, float& mx, float& scale) {
    mn = fmin_nan(mn, 1e30f);
    mx = fmax_nan(mx, -1e30f);
    scale = (mx - mn) / 3.0f + 1e-10f;
}

// Exact code of one element: clamp(round_half_away((x-min)/scale), 0, 3).
__device__ __forceinline__ uint32_t code_exact(float x, float mn, float scale) {
    float t = (x - mn) / scale;                  // correctly rounded
    float r = roundf(t);                         // half away from zero
    r = fminf(fmaxf(r, 0.0f), 3.0f);             // NaN -> 0
    return (uint32_t)r;
}

// Codes of four elements of one group.  Fast path: the quotient from a 1-ulp
// reciprocal differs from the correctly rounded one by < 1e-6 (t <= ~3), so
// unless u = t + 0.5 lies within kTieGuard of an integer the rounding
// decision is the same; any lane that is that close (or whose scale is outside
// the range where v_rcp_f32 is accurate) recomputes with the exact divide.
constexpr float kTieGuard = 4e-6f;

__device__ __forceinline__ uint32_t encode4(float x0, float x1, float x2, float x3,
                                            float mn, float scale) {
    const float r = __builtin_amdgcn_rcpf(scale);
    float u0 = fmaf(x0 - mn, r, 0.5f);
    float u1 = fmaf(x1 - mn, r, 0.5f);
    float u2 = fmaf(x2 - mn, r, 0.5f);
    float u3 = fmaf(x3 - mn, r, 0.5f);
    float d0 = fabsf(__builtin_amdgcn_fractf(u0) - 0.5f);
    float d1 = fabsf(__builtin_amdgcn_fractf(u1) - 0.5f);
    float d2 = fabsf(__builtin_amdgcn_fractf(u2) - 0.5f);
    float d3 = fabsf(__builtin_amdgcn_fractf(u3) - 0.5f);
    float dmax = fmaxf(fmaxf(d0, d1), fmaxf(d2, d3));
    const bool ok_scale = (scale >= 1e-10f) && (scale <= 0x1.0p120f);
    uint32_t q0, q1, q2, q3;
    if (__builtin_expect(!(dmax < 0.5f - kTieGuard) || !ok_scale, 0)) {
        // NaN dmax (a NaN quotient) also lands here; the exact path maps it to 0.
        q0 = code_exact(x0, mn, scale);
        q1 = code_exact(x1, mn, scale);
        q2 = code_exact(x2, mn, scale);
        q3 = code_exact(x3, mn, scale);
    } else {
        // fmaxf first so that a NaN element (whose NaN distance fmaxf dropped
        // above) still yields code 0, as the exact path does.
        q0 = (uint32_t)fminf(fmaxf(u0, 0.0f), 3.0f);
        q1 = (uint32_t)fminf(fmaxf(u1, 0.0f), 3.0f);
        q2 = (uint32_t)fminf(fmaxf(u2, 0.0f), 3.0f);
        q3 = (uint32_t)fminf(fmaxf(u3, 0.0f), 3.0f);
    }
    return q0 | (q1 << 2) | (q2 << 4) | (q3 << 6);
}

// ---------------------------------------------------------------------------
// K/V element types of new tokens and of the residual ring: 0 fp32, 1 bf16,
// 2 fp16 (the codes the C ABI takes).  16-bit values are widened exactly.
// ---------------------------------------------------------------------------
enum SrcType { kSrcF32 = 0, kSrcBF16 = 1, kSrcF16 = 2 };

__host__ __device__ constexpr int src_size(int dt) { return dt == kSrcF32 ? 4 : 2; }

template <int SRC>
__device__ __forceinline__ float widen(const void* p, int64_t i) {
    if constexpr (SRC == kSrcF32) {
        return static_cast<const float*>(p)[i];
    } else if constexpr (SRC == kSrcBF16) {
        return __uint_as_float((uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
    } else {
        return (float)static_cast<const _Float16*>(p)[i];
    }
}

// Elements i..i+3 widened to fp32 with one 16-byte (fp32) or 8-byte (16-bit)
// load: the offset must be aligned to that size.  The load is nontemporal: its
// callers (the flush reading K/V, the ring and new-token reads) stream data
// they read once, and keeping it out of L2 and the MALL measured 5-10 % faster
// for the batched prefill flush.
template <int SRC>
__device__ __forceinline__ float4 load4_vec(const void* p, int64_t i) {
    if constexpr (SRC == kSrcF32) {
        const kivi_f4v x = __builtin_nontemporal_load(
            reinterpret_cast<const kivi_f4v*>(static_cast<const float*>(p) + i));
        return make_float4(x.x, x.y, x.z, x.w);
    } else {
        const kivi_u2v w = __builtin_nontemporal_load(
            reinterpret_cast<const kivi_u2v*>(static_cast<const uint16_t*>(p) + i));
        const uint2 u = make_uint2(w.x, w.y);
        if constexpr (SRC == kSrcBF16) {
            return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                               __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
        } else {
            return make_float4((float)__builtin_bit_cast(_Float16, (uint16_t)(u.x & 0xffffu)),
                               (float)__builtin_bit_cast(_Float16, (uint16_t)(u.x >> 16)),
                               (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y & 0xffffu)),
                               (float)__builtin_bit_cast(_Float16, (uint16_t)(u.y >> 16)));
        }
    }
}

// Elements i..i+3 widened to fp32; `vec` selects the aligned single load.
template <int SRC>
__device__ __forceinline__ float4 load4_new(const void* p, int64_t i, bool vec) {
    if (vec) return load4_vec<SRC>(p, i);
    return make_float4(widen<SRC>(p, i), widen<SRC>(p, i + 1), widen<SRC>(p, i + 2),
                       widen<SRC>(p, i + 3));
}

// Elements i..i+3 of a 16-bit array widened to fp32, bf16 or fp16 chosen at
// run time by `half_mask` (all ones for fp16, 0 for bf16), after one 8-byte
// streaming load.  Both widenings are computed and merged by the mask: a
// select on a uniform flag is turned by the compiler into a branch per
// element, and each branch waits for every outstanding load (vmcnt(0)) --
// in the attention kernel, for the whole chunk prefetch ring (config 4 with
// a bf16 ring: 140 us against 106 us for an fp32 ring).
__device__ __forceinline__ float4 load4_16(const void* p, int64_t i, uint32_t half_mask) {
    const kivi_u2v w = __builtin_nontemporal_load(
        reinterpret_cast<const kivi_u2v*>(static_cast<const uint16_t*>(p) + i));
    auto cvt = [half_mask](uint32_t h) {       // h: the element in bits 15:0
        const uint32_t f = __float_as_uint((float)__builtin_bit_cast(_Float16, (uint16_t)h));
        return __uint_as_float((f & half_mask) | ((h << 16) & ~half_mask));
    };
    return make_float4(cvt(w.x & 0xffffu), cvt(w.x >> 16), cvt(w.y & 0xffffu), cvt(w.y >> 16));
}

// The same with the element type known at run time (a uniform branch; used
// on the residual ring, whose type follows the model's K/V).
__device__ __forceinline__ float4 load4_dt(const void* p, int64_t i, int dt) {
    if (dt == kSrcBF16) return load4_vec<kSrcBF16>(p, i);
    if (dt == kSrcF16) return load4_vec<kSrcF16>(p, i);
    return load4_vec<kSrcF32>(p, i);
}

__device__ __forceinline__ float load1_dt(const void* p, int64_t i, int dt) {
    if (dt == kSrcBF16) return widen<kSrcBF16>(p, i);
    if (dt == kSrcF16) return widen<kSrcF16>(p, i);
    return widen<kSrcF32>(p, i);
}

// x_hat = fl(fl(q * scale) + zero) (dequantize_kernels.cpp:24).
__device__ __forceinline__ float decode1(uint32_t q, float scale, float zero) {
    return __fadd_rn(__fmul_rn((float)q, scale), zero);
}

__device__ __forceinline__ float4 decode4(uint32_t byte, float scale, float zero) {
    float4 o;
    o.x = decode1(byte & 3u, scale, zero);
    o.y = decode1((byte >> 2) & 3u, scale, zero);
    o.z = decode1((byte >> 4) & 3u, scale, zero);
    o.w = decode1((byte >> 6) & 3u, scale, zero);
    return o;
}

// Streaming (nontemporal) stores for outputs written once and not read back
// by the same kernel: the lines go to HBM without being kept in L2 and the
// MALL.  For a write-dominated stream (dequantise writes 16 bytes per code
// byte read) this is the difference between ~4.8 and ~6.7 TB/s on MI355X.
__device__ __forceinline__ void store_stream(float4* p, const float4& v) {
    const kivi_f4v x = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(x, reinterpret_cast<kivi_f4v*>(p));
}
__device__ __forceinline__ void store_stream(float* p, float v) {
    __builtin_nontemporal_store(v, p);
}
__device__ __forceinline__ void store_stream(uint32_t* p, uint32_t v) {
    __builtin_nontemporal_store(v, p);
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every outstanding global load and store (s_waitcnt vmcnt(0)),
// which would drain a prefetch issued before the barrier.  Only for kernels
// where no thread reads global memory that another thread of the workgroup
// wrote.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace kivi
