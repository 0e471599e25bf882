// HBM-resident packed KV store: flush of the oldest residual tokens into 2-bit
// chunks.
//
// Replaces KiviCache._flush_group and the flush loop of add_tokens
// (src/kivi_sycl/cache/manager.py:242-249,309-374): instead of transposing on
// the host, copying to the device, round-tripping, copying back and
// concatenating a CPU history once per G tokens, one launch quantises every
// chunk a call owes, reading the tokens straight from where they are: the
// device residual ring first, then the caller's new-token tensor (any batch,
// head and token strides, fp32 / bf16 / fp16, channels contiguous).  It
// writes the packed chunks (and, optionally, the dequantised tokens the served
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
// store's own order (plain or MFMA-operand order).  bf16/fp16 inputs are
// widened exactly, so they quantise as their fp32 upcast does (the reference
// upcasts with .float(), manager.py:210-214).
#include <algorithm>

#include "kivi_common.hpp"
#include "../../include/kivi_hip.h"

namespace kivi {
namespace {

constexpr int kFlushBlock = 256;
constexpr int kTileMaxElems = 8192;   // G*D staged in LDS (fp32 tile + u8 codes)

struct FlushArgs {
    const void* k_res;    // [B, H, Rcap, D] ring of element type res_dt
    const void* v_res;
    const void* k_new;    // new tokens: element (b, h, t, d) at b*new_sb + h*new_sh + t*new_st + d
    const void* v_new;
    int64_t new_sb, new_sh, new_st;
    uint8_t* k_codes;     // [B, H, Cmax, G*D/4]
    float* k_scale;       // [B, H, Cmax, D]
    float* k_zero;
    uint8_t* v_codes;     // [B, H, Cmax, G*D/4]
    float* v_scale;       // [B, H, Cmax, D/Gv, G]
    float* v_zero;
    float* k_hist;        // optional [B, H, Tcap, D] dequantised keys
    float* v_hist;
    int64_t hist_cap;     // Tcap
    // Token vt of the flushed run is ring slot (res_start + vt) % Rcap while
    // vt < res_len, else new token vt - res_len.  Launch chunk j covers
    // tokens [j*G, (j+1)*G) and is stored as chunk `chunk + j`.
    int H, D, G, Gv, Rcap, res_start, res_len, Cmax, chunk;
    int n_chunks;         // chunks in this launch: run chunks first .. first+n_chunks-1
    int first;            // (flush_fast_kernel only; flush_kernel starts at 0)
    bool new_vec;         // new rows allow 16-byte (fp32) / 8-byte (16-bit) loads
    int res_dt;           // element type of the ring (SrcType)
};

// Where a flush_fast_kernel launch's chunks come from: all from the ring, all
// from the new tokens, or across both.
enum RunMode { kFromRing = 0, kFromNew = 1, kFromBoth = 2 };

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

// One workgroup per (b, kv-head, chunk).  TILE: the chunk's G x D tokens are
// first staged in LDS as fp32 with coalesced loads (needs G*D <=
// kTileMaxElems); otherwise elements are read from their source directly.
// SRC is the element type of the new-token source; the ring's is a.res_dt.
template <int LAYOUT, bool TILE, int SRC>
__global__ __launch_bounds__(kFlushBlock) void flush_kernel(FlushArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int D = a.D, G = a.G, Gv = a.Gv, NG = D / Gv;
    float* tile = reinterpret_cast<float*>(smem);                       // [G][D] if TILE
    uint8_t* codes = smem + (TILE ? (size_t)G * D * sizeof(float) : 0); // [G][D]
    const int bh = blockIdx.x;
    const int chunk = a.chunk + (int)blockIdx.y;
    const int vt0 = (int)blockIdx.y * G;            // first token of this chunk in the run
    const int64_t res_base = (int64_t)bh * a.Rcap * D;
    const int64_t new_base = (int64_t)(bh / a.H) * a.new_sb + (int64_t)(bh % a.H) * a.new_sh;
    const int64_t chunk_id = (int64_t)bh * a.Cmax + chunk;
    const int64_t code_bytes = (int64_t)G * D / 4;
    const int64_t hist_row0 = (int64_t)bh * a.hist_cap + (int64_t)chunk * G;

    auto stage = [&](const void* res, const void* nw) {
        const int nv = G * (D / 4);
        for (int e = threadIdx.x; e < nv; e += blockDim.x) {
            const int t = e / (D / 4), d4 = e % (D / 4);
            const int vt = vt0 + t;
            float4 x;
            if (vt < a.res_len) {
                x = load4_dt(res, res_base + (int64_t)ring(a.res_start, vt, a.Rcap) * D + 4 * d4,
                             a.res_dt);
            } else {
                x = load4_new<SRC>(nw, new_base + (int64_t)(vt - a.res_len) * a.new_st + 4 * d4,
                                   a.new_vec);
            }
            reinterpret_cast<float4*>(tile)[e] = x;
        }
    };
    auto elem = [&](const void* res, const void* nw, int t, int d) -> float {
        if constexpr (TILE) return tile[t * D + d];
        const int vt = vt0 + t;
        if (vt < a.res_len)
            return load1_dt(res, res_base + (int64_t)ring(a.res_start, vt, a.Rcap) * D + d, a.res_dt);
        return widen<SRC>(nw, new_base + (int64_t)(vt - a.res_len) * a.new_st + d);
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
        stage(a.k_res, a.k_new);
        __syncthreads();
    }
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float mn = 1e30f, mx = -1e30f;
        for (int t = 0; t < G; ++t) {
            const float x = elem(a.k_res, a.k_new, t, d);
            mn = fmin_nan(mn, x);
            mx = fmax_nan(mx, x);
        }
        float scale;
        finish_group(mn, mx, scale);
        a.k_scale[chunk_id * D + d] = scale;
        a.k_zero[chunk_id * D + d] = mn;
        for (int t = 0; t < G; ++t) {
            const uint32_t q = code_exact(elem(a.k_res, a.k_new, t, d), mn, scale);
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
        stage(a.v_res, a.v_new);
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
            const float x = elem(a.v_res, a.v_new, t, gi * Gv + j);
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
            const uint32_t q = code_exact(elem(a.v_res, a.v_new, t, d), mn, scale);
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

// RN(1/scale) (this library is built with correctly rounded division), or
// NaN when the scale lies outside [1e-10, 2^120], so that code_fast flags
// every element of that group for the exact path.
__device__ __forceinline__ float crcp_or_nan(float scale) {
    return (scale >= 1e-10f) && (scale <= 0x1.0p120f) ? 1.0f / scale : __builtin_nanf("");
}

// Code of one element from its group's min and y = crcp_or_nan(scale).
// u = fma(x - mn, y, 0.5 + kTieGuard) is within ~2 ulp of q + 0.5 +
// kTieGuard, where q = RN((x - mn) / scale); whenever fract(u) >= 2 kTieGuard,
// floor(u) = floor(q + 0.5), the code rounded half away from zero.  Otherwise
// (q within kTieGuard of a rounding tie, NaN input, flagged scale) `bad` is
// set and the caller recomputes the element with code_slow.  u <= 3.5 + 2
// kTieGuard when the code is kept, so no clamp is needed.
__device__ __forceinline__ uint32_t code_fast(float x, float mn, float y, bool& bad) {
    const float u = fmaf(x - mn, y, 0.5f + kTieGuard);
    bad |= !(__builtin_amdgcn_fractf(u) >= 2.0f * kTieGuard);
    return (uint32_t)u;
}

// Slow path of code_fast, exact without a divide for every accepted scale:
// with y = RN(1/s), q = RN(d*y) is within one ulp of d/s, the remainder
// d - q*s is exact under an FMA, and RN(q + (d - q*s)*y) = RN(d/s)
// (Markstein's theorem; d and s are normal and far from overflow for every
// scale crcp_or_nan accepts).  For that quotient q1 in [0, 3],
// (uint)(q1 + 0.5f) rounds half away from zero for every float except
// 0.5 - 2^-25, where adding 0.5 rounds up to 1.0; that one value is
// corrected.  A NaN input gives code 0, as code_exact does; a flagged scale
// (NaN y) goes to code_exact.  Bit-exact with code_exact
// (quantize_kernels.cpp:46-48, quant_tile.hpp:53-70) at about half its cost:
// bf16-grid inputs sit on rounding ties in ~40% of 64-lane waves.
__device__ __forceinline__ uint32_t code_slow(float x, float mn, float s, float y) {
    if (__builtin_isnan(y)) return code_exact(x, mn, s);
    const float d = x - mn;
    const float q = d * y;
    const float q1 = fmaf(fmaf(-q, s, d), y, q);
    const uint32_t c = (uint32_t)fmaxf(q1 + 0.5f, 0.0f);
    return c - (__float_as_uint(q1) == 0x3effffffu ? 1u : 0u);
}

// Matrix-core layout with compile-time shapes (G*D <= kTileMaxElems).  One
// workgroup of 256 threads per (b, kv-head, chunk) loads the chunk's K and V
// at once (V waits in registers while K is quantised).  Per tensor:
//  1. the [G][D] tokens go to an fp32 LDS tile whose rows are padded by four
//     floats; for values, rows 8..15 (mod 16) also hold their columns XORed
//     with 16, which makes the column reads of step 3 bank-conflict free (rows
//     8 apart would otherwise share banks) and keeps float4 groups whole;
//  2. group statistics: keys -- thread (segment s, channel d) scans tokens
//     [s*E, (s+1)*E) of channel d, segments combine through LDS; values --
//     thread (token t, group g, segment s) scans channels [g*GV + s*E, +E),
//     segments are adjacent lanes and combine with DPP.  Each group's
//     (min, scale, crcp_or_nan(scale)) is published in LDS (scale and zero
//     also go to HBM);
//  3. each thread builds whole output dwords of the matrix-core code order
//     (16 codes: two tiles x 8 elements) from the tile and the group
//     parameters and stores them straight to HBM, so codes never pass
//     through LDS as bytes.  Consecutive threads take consecutive lanes of
//     the same code word (64 lanes, then the next word), which spreads a
//     wave's tile reads over the banks.
// HIST: the dequantised history is also written (a template parameter, so
// that its test is not a branch per element).
// Same codes, scales, zeros and history as flush_kernel.
template <int G, int D, int GV, int SRC, int MODE, bool HIST>
__global__ __launch_bounds__(kFlushBlock) void flush_fast_kernel(FlushArgs a) {
    constexpr int N = G * D;
    constexpr int E = N / kFlushBlock;        // elements per thread in step 2
    constexpr int NG = D / GV;
    constexpr int NSK = kFlushBlock / D;
    constexpr int NSV = GV / E;
    constexpr int NV = N / 4 / kFlushBlock;   // float4 per thread per tensor
    constexpr int LD = D + 4;                 // padded tile row (floats)
    constexpr int NP = N / 1024;              // code dwords per lane per tensor
    constexpr int NW = (64 * NP + kFlushBlock - 1) / kFlushBlock;
    static_assert(N % (4 * kFlushBlock) == 0 && E * NSK == G && NSV >= 1 && NSV <= 64 &&
                  (NSV & (NSV - 1)) == 0 && kFlushBlock % D == 0 && G % 16 == 0 &&
                  GV % 32 == 0, "flush_fast shape");
    __shared__ __align__(16) float tile[G * LD];
    __shared__ __align__(16) float kpar[3][D];          // min, scale, 1/scale per channel
    // (min, scale, 1/scale, -) per value group, token-major with one pad
    // float4 after every 8 tokens: the code pass's lanes read 4 token rows 8
    // apart at once, which then fall in distinct banks.
    __shared__ __align__(16) float4 vpar[G * NG + G / 8];
    auto vpi = [](int t, int g) { return t * NG + g + t / 8; };
    __shared__ float part[2][NSK][D];
    // fp32 sources (latency-bound) stage a tensor's code words in LDS and
    // store each lane's NP words as one 16-byte run: 228 -> 220 us for the
    // config-2 fp32 prompt; 16-bit sources (VALU-bound) store each word
    // where it is made (the extra barrier cost them 138 -> 142 us).
    constexpr bool kStageCodes = SRC == kSrcF32 && NP % 4 == 0;
    __shared__ __align__(16) uint32_t cbuf[kStageCodes ? 64 * NP : 4];
    auto put_word = [&](uint32_t* dst, int l, int w, uint32_t word) {
        if constexpr (kStageCodes) cbuf[l * NP + w] = word;
        else dst[l * NP + w] = word;
    };
    auto flush_codes = [&](uint32_t* dst) {
        if constexpr (kStageCodes) {
            lds_barrier();
            for (int e = (int)threadIdx.x; e < 16 * NP; e += kFlushBlock)
                reinterpret_cast<uint4*>(dst)[e] = reinterpret_cast<const uint4*>(cbuf)[e];
        }
    };

    const int tid = threadIdx.x;
    const int bh = blockIdx.x;
    const int64_t res_base = (int64_t)bh * a.Rcap * D;
    const int64_t new_base = (int64_t)(bh / a.H) * a.new_sb + (int64_t)(bh % a.H) * a.new_sh;
    const int j = a.first + (int)blockIdx.y;   // run chunk of this workgroup

    // K or V of run chunk j: float4 slot i*256 + tid of the [G][D] chunk.  The
    // source is fixed per launch (MODE), so the loads carry no branches.  SRC
    // is the element type of that source: the ring's for kFromRing, the new
    // tokens' otherwise (kFromBoth reads its ring part by a.res_dt).
    auto load = [&](float4 (&x)[NV], const void* res, const void* nw, int j) {
        const int vt0 = j * G;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e = i * kFlushBlock + tid;
            const int t = e / (D / 4), d4 = e % (D / 4);
            const int vt = vt0 + t;
            if constexpr (MODE == kFromNew) {
                x[i] = load4_vec<SRC>(nw, new_base + (int64_t)(vt - a.res_len) * a.new_st + 4 * d4);
            } else if constexpr (MODE == kFromRing) {
                const int64_t row = res_base + (int64_t)ring(a.res_start, vt, a.Rcap) * D;
                x[i] = load4_vec<SRC>(res, row + 4 * d4);
            } else {
                if (vt < a.res_len) {
                    const int64_t row = res_base + (int64_t)ring(a.res_start, vt, a.Rcap) * D;
                    x[i] = load4_dt(res, row + 4 * d4, a.res_dt);
                } else {
                    x[i] = load4_vec<SRC>(nw, new_base + (int64_t)(vt - a.res_len) * a.new_st + 4 * d4);
                }
            }
        }
    };
    // Tile offset of (token t, channel c): keys plain, values with the
    // channel XORed with 16 in rows 8..15 (mod 16).
    auto kat = [](int t, int c) { return t * LD + c; };
    auto vat = [](int t, int c) { return t * LD + (c ^ (16 * ((t >> 3) & 1))); };
    auto put = [&](const float4 (&x)[NV], auto at) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e = i * kFlushBlock + tid;
            const int t = e / (D / 4), d4 = e % (D / 4);
            *reinterpret_cast<float4*>(tile + at(t, 4 * d4)) = x[i];
        }
    };
    // Dequantised tokens (written back into the tile) -> history rows.
    auto copy_hist = [&](float* hist, int64_t row0, auto at) {
        for (int e = tid; e < N / 4; e += kFlushBlock) {
            const int t = e / (D / 4), d4 = e % (D / 4);
            reinterpret_cast<float4*>(hist + (row0 + t) * D)[d4] =
                *reinterpret_cast<const float4*>(tile + at(t, 4 * d4));
        }
    };

    float4 kx[NV], vx[NV];
    load(kx, a.k_res, a.k_new, j);
    load(vx, a.v_res, a.v_new, j);
    {
        const int chunk = a.chunk + j;
        const int64_t chunk_id = (int64_t)bh * a.Cmax + chunk;
        const int64_t hist_row0 = (int64_t)bh * a.hist_cap + (int64_t)chunk * G;
        uint32_t* const kout = reinterpret_cast<uint32_t*>(a.k_codes + chunk_id * (N / 4));
        uint32_t* const vout = reinterpret_cast<uint32_t*>(a.v_codes + chunk_id * (N / 4));

        // ================================ keys ================================
        put(kx, kat);
        lds_barrier();
        {
            const int d = tid % D, sg = tid / D;
            float mn = 1e30f, mx = -1e30f;
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const float x = tile[(sg * E + i) * LD + d];
                mn = fmin_nan(mn, x);
                mx = fmax_nan(mx, x);
            }
            if constexpr (NSK > 1) {
                part[0][sg][d] = mn;
                part[1][sg][d] = mx;
                lds_barrier();
#pragma unroll
                for (int s2 = 0; s2 < NSK; ++s2) {
                    mn = fmin_nan(mn, part[0][s2][d]);
                    mx = fmax_nan(mx, part[1][s2][d]);
                }
            }
            float scale;
            finish_group(mn, mx, scale);
            if (sg == 0) {
                a.k_scale[chunk_id * D + d] = scale;
                a.k_zero[chunk_id * D + d] = mn;
                kpar[0][d] = mn;
                kpar[1][d] = scale;
                kpar[2][d] = crcp_or_nan(scale);
            }
        }
        lds_barrier();
        // Key tile ks*(G/16)+nb: lane l element j = token 16nb + l%16, channel
        // 32ks + 8(l/16) + j.  Dword (l, w) holds tiles 2w and 2w+1.
#pragma unroll
        for (int it = 0; it < NW; ++it) {
            const int e = it * kFlushBlock + tid;
            if (e < 64 * NP) {
                const int l = e % 64, w = e / 64;
                uint32_t word = 0;
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const int tl = 2 * w + m, ks = tl / (G / 16), nb = tl % (G / 16);
                    const int t = 16 * nb + l % 16, d0 = 32 * ks + 8 * (l / 16);
                    float x[8], mnv[8], scv[8], rcv[8];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float4 f = *reinterpret_cast<const float4*>(tile + t * LD + d0 + 4 * h);
                        const float4 pm = *reinterpret_cast<const float4*>(&kpar[0][d0 + 4 * h]);
                        const float4 ps = *reinterpret_cast<const float4*>(&kpar[1][d0 + 4 * h]);
                        const float4 pr = *reinterpret_cast<const float4*>(&kpar[2][d0 + 4 * h]);
                        x[4 * h] = f.x; x[4 * h + 1] = f.y; x[4 * h + 2] = f.z; x[4 * h + 3] = f.w;
                        mnv[4 * h] = pm.x; mnv[4 * h + 1] = pm.y; mnv[4 * h + 2] = pm.z; mnv[4 * h + 3] = pm.w;
                        scv[4 * h] = ps.x; scv[4 * h + 1] = ps.y; scv[4 * h + 2] = ps.z; scv[4 * h + 3] = ps.w;
                        rcv[4 * h] = pr.x; rcv[4 * h + 1] = pr.y; rcv[4 * h + 2] = pr.z; rcv[4 * h + 3] = pr.w;
                    }
                    // An element near a rounding tie is resolved on its own,
                    // so a wave pays the slow path only for the element
                    // positions where some lane needs it.
                    uint32_t q[8];
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        bool bad = false;
                        q[jj] = code_fast(x[jj], mnv[jj], rcv[jj], bad);
                        if (__builtin_expect(bad, 0)) q[jj] = code_slow(x[jj], mnv[jj], scv[jj], rcv[jj]);
                    }
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        word |= q[jj] << mfma_code_bit(m, jj);
                        if constexpr (HIST) tile[t * LD + d0 + jj] = decode1(q[jj], scv[jj], mnv[jj]);
                    }
                }
                put_word(kout, l, w, word);
            }
        }
        flush_codes(kout);
        if constexpr (HIST) {
            lds_barrier();
            copy_hist(a.k_hist, hist_row0, kat);
        }

        // =============================== values ===============================
        lds_barrier();
        put(vx, vat);
        lds_barrier();
        {
            const int sg = tid % NSV, grp = tid / NSV;
            const int t = grp / NG, gi = grp % NG;
            const int c0 = gi * GV + sg * E;
            float mn = 1e30f, mx = -1e30f;
#pragma unroll
            for (int q4 = 0; q4 < E / 4; ++q4) {
                const float4 f = *reinterpret_cast<const float4*>(tile + vat(t, c0 + 4 * q4));
                mn = fmin_nan(fmin_nan(mn, f.x), fmin_nan(f.y, fmin_nan(f.z, f.w)));
                mx = fmax_nan(fmax_nan(mx, f.x), fmax_nan(f.y, fmax_nan(f.z, f.w)));
            }
            seg_min_max<NSV>(mn, mx);
            float scale;
            finish_group(mn, mx, scale);
            if (sg == 0) {
                a.v_scale[(chunk_id * NG + gi) * G + t] = scale;
                a.v_zero[(chunk_id * NG + gi) * G + t] = mn;
                vpar[vpi(t, gi)] = make_float4(mn, scale, crcp_or_nan(scale), 0.0f);
            }
        }
        lds_barrier();
        // Value tile kt*(D/16)+nb: lane l element j = token 32kt + 8(l/16) + j,
        // channel 16nb + l%16.
#pragma unroll
        for (int it = 0; it < NW; ++it) {
            const int e = it * kFlushBlock + tid;
            if (e < 64 * NP) {
                const int l = e % 64, w = e / 64;
                uint32_t word = 0;
#pragma unroll
                for (int m = 0; m < 2; ++m) {
                    const int tl = 2 * w + m, kt = tl / (D / 16), nb = tl % (D / 16);
                    const int c = 16 * nb + l % 16, t0 = 32 * kt + 8 * (l / 16);
                    float x[8];
                    float4 par[8];
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        x[jj] = tile[vat(t0 + jj, c)];
                        par[jj] = vpar[vpi(t0 + jj, c / GV)];
                    }
                    uint32_t q[8];
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        bool bad = false;
                        q[jj] = code_fast(x[jj], par[jj].x, par[jj].z, bad);
                        if (__builtin_expect(bad, 0))
                            q[jj] = code_slow(x[jj], par[jj].x, par[jj].y, par[jj].z);
                    }
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        word |= q[jj] << mfma_code_bit(m, jj);
                        if constexpr (HIST) tile[vat(t0 + jj, c)] = decode1(q[jj], par[jj].y, par[jj].x);
                    }
                }
                put_word(vout, l, w, word);
            }
        }
        flush_codes(vout);
        if constexpr (HIST) {
            lds_barrier();
            copy_hist(a.v_hist, hist_row0, vat);
        }
    }
}

template <int G, int D, int GV, int MODE, bool HIST>
void launch_fast5(const FlushArgs& a, int src, dim3 grid, hipStream_t st) {
    switch (src) {
        case kSrcBF16: flush_fast_kernel<G, D, GV, kSrcBF16, MODE, HIST><<<grid, kFlushBlock, 0, st>>>(a); break;
        case kSrcF16: flush_fast_kernel<G, D, GV, kSrcF16, MODE, HIST><<<grid, kFlushBlock, 0, st>>>(a); break;
        default: flush_fast_kernel<G, D, GV, kSrcF32, MODE, HIST><<<grid, kFlushBlock, 0, st>>>(a); break;
    }
}

template <int G, int D, int GV, int MODE>
void launch_fast4(const FlushArgs& a, int src, dim3 grid, hipStream_t st) {
    if (a.k_hist) launch_fast5<G, D, GV, MODE, true>(a, src, grid, st);
    else launch_fast5<G, D, GV, MODE, false>(a, src, grid, st);
}

template <int G, int D, int GV>
void launch_fast3(const FlushArgs& a, int src, int mode, dim3 grid, hipStream_t st) {
    if (mode == kFromNew) launch_fast4<G, D, GV, kFromNew>(a, src, grid, st);
    else if (mode == kFromRing) launch_fast4<G, D, GV, kFromRing>(a, a.res_dt, grid, st);
    else launch_fast4<G, D, GV, kFromBoth>(a, src, grid, st);
}

template <int G, int D>
bool launch_fast2(const FlushArgs& a, int src, int mode, dim3 grid, hipStream_t st) {
    switch (a.Gv) {
        case 32: launch_fast3<G, D, 32>(a, src, mode, grid, st); return true;
        case 64: launch_fast3<G, D, 64>(a, src, mode, grid, st); return true;
        case 128:
            if constexpr (D >= 128) { launch_fast3<G, D, 128>(a, src, mode, grid, st); return true; }
            return false;
        case 256:
            if constexpr (D >= 256) { launch_fast3<G, D, 256>(a, src, mode, grid, st); return true; }
            return false;
        default: return false;
    }
}

bool fast_shape(int G, int D) {
    return (G == 32 && (D == 64 || D == 128 || D == 256)) || (G == 64 && (D == 64 || D == 128));
}

// One flush_fast_kernel launch over run chunks [first, first + count) whose
// source is `mode`: one workgroup per (b, kv-head, chunk).
bool launch_fast(FlushArgs a, int src, int mode, int first, int count, int bh, hipStream_t st) {
    a.first = first;
    a.n_chunks = count;
    const dim3 grid(bh, count);
    if (a.G == 32 && a.D == 64) return launch_fast2<32, 64>(a, src, mode, grid, st);
    if (a.G == 32 && a.D == 128) return launch_fast2<32, 128>(a, src, mode, grid, st);
    if (a.G == 32 && a.D == 256) return launch_fast2<32, 256>(a, src, mode, grid, st);
    if (a.G == 64 && a.D == 64) return launch_fast2<64, 64>(a, src, mode, grid, st);
    if (a.G == 64 && a.D == 128) return launch_fast2<64, 128>(a, src, mode, grid, st);
    return false;
}

template <int LAYOUT, bool TILE>
void launch_flush(const FlushArgs& a, int src, dim3 grid, size_t lds, hipStream_t st) {
    switch (src) {
        case kSrcBF16: flush_kernel<LAYOUT, TILE, kSrcBF16><<<grid, kFlushBlock, lds, st>>>(a); break;
        case kSrcF16: flush_kernel<LAYOUT, TILE, kSrcF16><<<grid, kFlushBlock, lds, st>>>(a); break;
        default: flush_kernel<LAYOUT, TILE, kSrcF32><<<grid, kFlushBlock, lds, st>>>(a); break;
    }
}

// Residual append: token t of the new K/V goes to ring slot (slot + t) % Rcap
// of every (b, kv-head), four channels per thread, K and V in the same
// launch.  An fp32 ring (RES == kSrcF32) takes any source type, widened; a
// 16-bit ring takes its own type only, copied bit for bit.
struct AppendArgs {
    const void* k_new;
    const void* v_new;
    int64_t sb, sh, st;            // element strides of the new tokens (channels contiguous)
    void* k_res;                   // [B, H, Rcap, D]
    void* v_res;
    int64_t total;                 // B * H * n * D/4
    int H, D, n, Rcap, slot;
    bool vec;
};

// Four raw 16-bit elements at i..i+3 (one 8-byte load when `vec`).
__device__ __forceinline__ uint2 load4_raw16(const void* p, int64_t i, bool vec) {
    const uint16_t* h = static_cast<const uint16_t*>(p) + i;
    if (vec) return *reinterpret_cast<const uint2*>(h);
    return make_uint2((uint32_t)h[0] | ((uint32_t)h[1] << 16), (uint32_t)h[2] | ((uint32_t)h[3] << 16));
}

// Element quad i of one append (i < a.total).
template <int SRC, int RES>
__device__ __forceinline__ void append_quad(const AppendArgs& a, int64_t i) {
    const int d4n = a.D / 4;
    const int d4 = (int)(i % d4n);
    const int64_t r = i / d4n;
    const int t = (int)(r % a.n);
    const int64_t bh = r / a.n;
    const int64_t off = (bh / a.H) * a.sb + (bh % a.H) * a.sh + (int64_t)t * a.st + 4 * d4;
    int s = a.slot + t;
    s = s >= a.Rcap ? s - a.Rcap : s;
    const int64_t dst = (bh * a.Rcap + s) * a.D / 4 + d4;
    if constexpr (RES == kSrcF32) {
        reinterpret_cast<float4*>(a.k_res)[dst] = load4_new<SRC>(a.k_new, off, a.vec);
        reinterpret_cast<float4*>(a.v_res)[dst] = load4_new<SRC>(a.v_new, off, a.vec);
    } else {
        static_assert(RES == SRC, "a 16-bit ring takes its own element type");
        reinterpret_cast<uint2*>(a.k_res)[dst] = load4_raw16(a.k_new, off, a.vec);
        reinterpret_cast<uint2*>(a.v_res)[dst] = load4_raw16(a.v_new, off, a.vec);
    }
}

template <int SRC, int RES>
__global__ __launch_bounds__(256) void append_kernel(AppendArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < a.total) append_quad<SRC, RES>(a, i);
}

// Several layers' appends in one launch (blockIdx.y = layer within the
// launch): the per-layer pointers, strides and slots travel in the kernel
// arguments, the shapes are shared.
constexpr int kMaxAppendLayers = 16;

struct AppendLayer {
    const void* k_new;
    const void* v_new;
    int64_t sb, sh, st;
    void* k_res;
    void* v_res;
    int slot;
    bool vec;
};

struct AppendLayers {
    AppendLayer layer[kMaxAppendLayers];
    int64_t total;                 // B * H * n * D/4 per layer
    int H, D, n, Rcap;
};

template <int SRC, int RES>
__global__ __launch_bounds__(256) void append_layers_kernel(AppendLayers a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= a.total) return;
    const AppendLayer& l = a.layer[blockIdx.y];
    const AppendArgs one{l.k_new, l.v_new, l.sb, l.sh, l.st, l.k_res, l.v_res, a.total, a.H,
                         a.D, a.n, a.Rcap, l.slot, l.vec};
    append_quad<SRC, RES>(one, i);
}

}  // namespace
}  // namespace kivi

using namespace kivi;

extern "C" int kivi_store_code_layout(int32_t head_dim, int32_t group_size_k,
                                      int32_t group_size_v) {
    return code_layout_for(head_dim, group_size_k, group_size_v);
}

extern "C" int kivi_store_flush_chunks(
        const void* k_res, const void* v_res, int32_t res_dtype, const void* k_new, const void* v_new,
        int32_t new_dtype, int64_t new_batch_stride, int64_t new_head_stride,
        int64_t new_token_stride, int32_t new_tokens, uint8_t* k_codes, float* k_scale,
        float* k_zero, uint8_t* v_codes, float* v_scale, float* v_zero, float* k_hist,
        float* v_hist, int64_t hist_capacity, int32_t batch, int32_t kv_heads,
        int32_t head_dim, int32_t group_size_k, int32_t group_size_v, int32_t res_capacity,
        int32_t res_start, int32_t res_len, int32_t chunk_capacity, int32_t chunk_index,
        int32_t n_chunks, void* stream) {
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
    if (res_len < 0 || res_len > res_capacity)
        return set_error(kErrInvalidArgument, "res_len %d outside [0, %d]", res_len,
                         res_capacity);
    if (new_tokens < 0 || (new_tokens > 0 && (!k_new || !v_new)))
        return set_error(kErrInvalidArgument, "new tokens given without k_new/v_new");
    if (new_dtype < kSrcF32 || new_dtype > kSrcF16)
        return set_error(kErrInvalidArgument, "new_dtype %d is not 0 (f32), 1 (bf16) or 2 (f16)",
                         new_dtype);
    if (res_dtype < kSrcF32 || res_dtype > kSrcF16)
        return set_error(kErrInvalidArgument, "res_dtype %d is not 0 (f32), 1 (bf16) or 2 (f16)",
                         res_dtype);
    if (new_batch_stride < 0 || new_head_stride < 0 || new_token_stride < 0)
        return set_error(kErrInvalidArgument, "negative new-token strides");
    if (n_chunks <= 0 || n_chunks > 65535)
        return set_error(kErrInvalidArgument, "n_chunks %d outside [1, 65535]", n_chunks);
    if ((int64_t)n_chunks * group_size_k > (int64_t)res_len + new_tokens)
        return set_error(kErrInvalidArgument, "%d chunks of %d need %lld tokens, %lld available",
                         n_chunks, group_size_k, (long long)n_chunks * group_size_k,
                         (long long)res_len + new_tokens);
    if (chunk_index < 0 || (int64_t)chunk_index + n_chunks > chunk_capacity)
        return set_error(kErrInvalidArgument, "chunks %d..%d outside capacity %d", chunk_index,
                         chunk_index + n_chunks - 1, chunk_capacity);
    if (k_hist && (int64_t)(chunk_index + n_chunks) * group_size_k > hist_capacity)
        return set_error(kErrInvalidArgument, "history capacity %lld too small",
                         (long long)hist_capacity);
    const int64_t elems = (int64_t)group_size_k * head_dim;
    if (elems > 64 * 1024)
        return set_error(kErrUnsupported, "group_size_k * head_dim = %lld exceeds 65536",
                         (long long)elems);
    const bool aligned = ((uintptr_t)k_res % 16 == 0) && ((uintptr_t)v_res % 16 == 0) &&
                         (!k_hist || ((uintptr_t)k_hist % 16 == 0 && (uintptr_t)v_hist % 16 == 0));
    const int esize = new_dtype == kSrcF32 ? 4 : 2;
    const int64_t vec_bytes = 4 * esize;   // four channels per load
    const bool new_vec = new_tokens == 0 ||
        ((uintptr_t)k_new % vec_bytes == 0 && (uintptr_t)v_new % vec_bytes == 0 &&
         (new_batch_stride * esize) % vec_bytes == 0 && (new_head_stride * esize) % vec_bytes == 0 &&
         (new_token_stride * esize) % vec_bytes == 0);
    const bool tile = elems <= kTileMaxElems && aligned;
    const int layout = code_layout_for(head_dim, group_size_k, group_size_v);
    const size_t lds = (size_t)elems * (tile ? sizeof(float) + 1 : 1);
    FlushArgs a{k_res, v_res, k_new, v_new, new_batch_stride, new_head_stride,
                new_token_stride, k_codes, k_scale, k_zero, v_codes, v_scale, v_zero,
                k_hist, v_hist, hist_capacity, kv_heads, head_dim, group_size_k,
                group_size_v, res_capacity, res_start, res_len, chunk_capacity, chunk_index,
                n_chunks, 0, new_vec, res_dtype};
    const dim3 grid(batch * kv_heads, n_chunks);
    hipStream_t st = (hipStream_t)stream;
    const bool fast_gv = group_size_v % 32 == 0 && group_size_v <= head_dim;
    if (layout == kLayoutMfma && tile && new_vec && fast_gv &&
        fast_shape(group_size_k, head_dim)) {
        // Chunks wholly in the ring, at most one across ring and new tokens,
        // then chunks wholly in the new tokens: one launch each.
        const int bh = batch * kv_heads;
        const int n_ring = std::min(n_chunks, res_len / group_size_k);
        const int n_both = (n_ring < n_chunks && res_len % group_size_k) ? 1 : 0;
        const int n_new = n_chunks - n_ring - n_both;
        if (n_ring) launch_fast(a, new_dtype, kFromRing, 0, n_ring, bh, st);
        if (n_both) launch_fast(a, new_dtype, kFromBoth, n_ring, 1, bh, st);
        if (n_new) launch_fast(a, new_dtype, kFromNew, n_ring + n_both, n_new, bh, st);
        return check_launch("store_flush");
    }
    if (layout == kLayoutMfma) {
        if (tile) launch_flush<kLayoutMfma, true>(a, new_dtype, grid, lds, st);
        else launch_flush<kLayoutMfma, false>(a, new_dtype, grid, lds, st);
    } else {
        if (tile) launch_flush<kLayoutPlain, true>(a, new_dtype, grid, lds, st);
        else launch_flush<kLayoutPlain, false>(a, new_dtype, grid, lds, st);
    }
    return check_launch("store_flush");
}

extern "C" int kivi_store_flush(const void* k_res, const void* v_res, int32_t res_dtype,
                                uint8_t* k_codes,
                                float* k_scale, float* k_zero, uint8_t* v_codes,
                                float* v_scale, float* v_zero, float* k_hist, float* v_hist,
                                int64_t hist_capacity, int32_t batch, int32_t kv_heads,
                                int32_t head_dim, int32_t group_size_k,
                                int32_t group_size_v, int32_t res_capacity,
                                int32_t res_start, int32_t chunk_capacity,
                                int32_t chunk_index, void* stream) {
    return kivi_store_flush_chunks(k_res, v_res, res_dtype, nullptr, nullptr, kSrcF32, 0, 0, 0, 0,
                                   k_codes, k_scale, k_zero, v_codes, v_scale, v_zero, k_hist,
                                   v_hist, hist_capacity, batch, kv_heads, head_dim,
                                   group_size_k, group_size_v, res_capacity, res_start,
                                   group_size_k, chunk_capacity, chunk_index, 1, stream);
}

extern "C" int kivi_store_append(const void* k_new, const void* v_new, int32_t new_dtype,
                                 int64_t new_batch_stride, int64_t new_head_stride,
                                 int64_t new_token_stride, int32_t new_tokens, void* k_res,
                                 void* v_res, int32_t res_dtype, int32_t batch, int32_t kv_heads,
                                 int32_t head_dim, int32_t res_capacity, int32_t slot,
                                 void* stream) {
    if (!k_new || !v_new || !k_res || !v_res)
        return set_error(kErrInvalidArgument, "null tensor pointer");
    if (batch <= 0 || kv_heads <= 0)
        return set_error(kErrInvalidArgument, "batch and kv_heads must be positive");
    if (head_dim <= 0 || head_dim % 4)
        return set_error(kErrInvalidArgument, "head_dim must be positive and divisible by 4");
    if (new_dtype < kSrcF32 || new_dtype > kSrcF16)
        return set_error(kErrInvalidArgument, "new_dtype %d is not 0 (f32), 1 (bf16) or 2 (f16)",
                         new_dtype);
    if (res_dtype != kSrcF32 && res_dtype != new_dtype)
        return set_error(kErrInvalidArgument,
                         "res_dtype %d: the ring is f32 (0) or of the new tokens' type (%d)",
                         res_dtype, new_dtype);
    if (new_batch_stride < 0 || new_head_stride < 0 || new_token_stride < 0)
        return set_error(kErrInvalidArgument, "negative new-token strides");
    if (res_capacity <= 0 || slot < 0 || slot >= res_capacity)
        return set_error(kErrInvalidArgument, "slot %d outside [0, %d)", slot, res_capacity);
    if (new_tokens < 0 || new_tokens > res_capacity)
        return set_error(kErrInvalidArgument, "%d new tokens exceed the ring capacity %d",
                         new_tokens, res_capacity);
    if ((uintptr_t)k_res % 16 || (uintptr_t)v_res % 16)
        return set_error(kErrInvalidArgument, "residual ring must be 16-byte aligned");
    if (new_tokens == 0) return 0;
    const int esize = new_dtype == kSrcF32 ? 4 : 2;
    const int64_t vb = 4 * esize;
    const bool vec = (uintptr_t)k_new % vb == 0 && (uintptr_t)v_new % vb == 0 &&
                     (new_batch_stride * esize) % vb == 0 && (new_head_stride * esize) % vb == 0 &&
                     (new_token_stride * esize) % vb == 0;
    AppendArgs a{k_new, v_new, new_batch_stride, new_head_stride, new_token_stride, k_res, v_res,
                 (int64_t)batch * kv_heads * new_tokens * (head_dim / 4), kv_heads, head_dim,
                 new_tokens, res_capacity, slot, vec};
    const unsigned grid = (unsigned)((a.total + 255) / 256);
    hipStream_t st = (hipStream_t)stream;
    if (res_dtype == kSrcBF16) {
        append_kernel<kSrcBF16, kSrcBF16><<<grid, 256, 0, st>>>(a);
    } else if (res_dtype == kSrcF16) {
        append_kernel<kSrcF16, kSrcF16><<<grid, 256, 0, st>>>(a);
    } else {
        switch (new_dtype) {
            case kSrcBF16: append_kernel<kSrcBF16, kSrcF32><<<grid, 256, 0, st>>>(a); break;
            case kSrcF16: append_kernel<kSrcF16, kSrcF32><<<grid, 256, 0, st>>>(a); break;
            default: append_kernel<kSrcF32, kSrcF32><<<grid, 256, 0, st>>>(a); break;
        }
    }
    return check_launch("store_append");
}

extern "C" int kivi_store_append_layers(int32_t n_layers, const void* const* k_new,
                                        const void* const* v_new, const int64_t* new_strides,
                                        int32_t new_dtype, int32_t new_tokens,
                                        void* const* k_res, void* const* v_res,
                                        int32_t res_dtype, int32_t batch, int32_t kv_heads,
                                        int32_t head_dim, int32_t res_capacity,
                                        const int32_t* slots, void* stream) {
    if (n_layers < 0) return set_error(kErrInvalidArgument, "n_layers %d < 0", n_layers);
    if (n_layers == 0 || new_tokens == 0) return 0;
    if (!k_new || !v_new || !new_strides || !k_res || !v_res || !slots)
        return set_error(kErrInvalidArgument, "null layer array");
    if (batch <= 0 || kv_heads <= 0)
        return set_error(kErrInvalidArgument, "batch and kv_heads must be positive");
    if (head_dim <= 0 || head_dim % 4)
        return set_error(kErrInvalidArgument, "head_dim must be positive and divisible by 4");
    if (new_dtype < kSrcF32 || new_dtype > kSrcF16)
        return set_error(kErrInvalidArgument, "new_dtype %d is not 0 (f32), 1 (bf16) or 2 (f16)",
                         new_dtype);
    if (res_dtype != kSrcF32 && res_dtype != new_dtype)
        return set_error(kErrInvalidArgument,
                         "res_dtype %d: the ring is f32 (0) or of the new tokens' type (%d)",
                         res_dtype, new_dtype);
    if (res_capacity <= 0 || new_tokens < 0 || new_tokens > res_capacity)
        return set_error(kErrInvalidArgument, "%d new tokens exceed the ring capacity %d",
                         new_tokens, res_capacity);
    const int esize = new_dtype == kSrcF32 ? 4 : 2;
    const int64_t vb = 4 * esize;
    AppendLayers a{};
    a.total = (int64_t)batch * kv_heads * new_tokens * (head_dim / 4);
    a.H = kv_heads;
    a.D = head_dim;
    a.n = new_tokens;
    a.Rcap = res_capacity;
    hipStream_t st = (hipStream_t)stream;
    for (int l0 = 0; l0 < n_layers; l0 += kMaxAppendLayers) {
        const int nl = n_layers - l0 < kMaxAppendLayers ? n_layers - l0 : kMaxAppendLayers;
        for (int j = 0; j < nl; ++j) {
            const int l = l0 + j;
            const int64_t* str = new_strides + 3 * (int64_t)l;
            if (!k_new[l] || !v_new[l] || !k_res[l] || !v_res[l])
                return set_error(kErrInvalidArgument, "null tensor pointer (layer %d)", l);
            if (str[0] < 0 || str[1] < 0 || str[2] < 0)
                return set_error(kErrInvalidArgument, "negative new-token strides (layer %d)", l);
            if (slots[l] < 0 || slots[l] >= res_capacity)
                return set_error(kErrInvalidArgument, "slot %d outside [0, %d) (layer %d)",
                                 slots[l], res_capacity, l);
            if ((uintptr_t)k_res[l] % 16 || (uintptr_t)v_res[l] % 16)
                return set_error(kErrInvalidArgument,
                                 "residual ring must be 16-byte aligned (layer %d)", l);
            AppendLayer& e = a.layer[j];
            e.k_new = k_new[l];
            e.v_new = v_new[l];
            e.sb = str[0];
            e.sh = str[1];
            e.st = str[2];
            e.k_res = k_res[l];
            e.v_res = v_res[l];
            e.slot = slots[l];
            e.vec = (uintptr_t)k_new[l] % vb == 0 && (uintptr_t)v_new[l] % vb == 0 &&
                    (str[0] * esize) % vb == 0 && (str[1] * esize) % vb == 0 &&
                    (str[2] * esize) % vb == 0;
        }
        const dim3 grid((unsigned)((a.total + 255) / 256), (unsigned)nl);
        if (res_dtype == kSrcBF16) {
            append_layers_kernel<kSrcBF16, kSrcBF16><<<grid, 256, 0, st>>>(a);
        } else if (res_dtype == kSrcF16) {
            append_layers_kernel<kSrcF16, kSrcF16><<<grid, 256, 0, st>>>(a);
        } else {
            switch (new_dtype) {
                case kSrcBF16: append_layers_kernel<kSrcBF16, kSrcF32><<<grid, 256, 0, st>>>(a); break;
                case kSrcF16: append_layers_kernel<kSrcF16, kSrcF32><<<grid, 256, 0, st>>>(a); break;
                default: append_layers_kernel<kSrcF32, kSrcF32><<<grid, 256, 0, st>>>(a); break;
            }
        }
        const int rc = check_launch("store_append_layers");
        if (rc) return rc;
    }
    return 0;
}
