// Fused packed-KV decode attention for gfx950.
//
// No reference counterpart: the reference dequantises every flushed chunk back
// to an fp32 CPU history (src/kivi_sycl/cache/manager.py:362-374) and lets the
// HF model run ordinary attention over [history || residual]
// (manager.py:251-290; the math it relies on is stated in
// tests/integration/test_attention_fix.py:40-43,91-93).  This kernel computes
//   o[h] = softmax(q[h] . [K_hat ; K_res]^T * scale) . [V_hat ; V_res]
// for one query token per sequence directly from the packed store
// (kivi_store.hip layout) and the fp32 residual ring, without materialising
// K_hat / V_hat.  Query head h reads kv head h / (Hq / Hkv) (HF repeat_kv).
//
// Dequantisation is factored out of the inner loops:
//   q . k_hat(t) = sum_d (q_d * ks_d) * code_dt + sum_d q_d * kz_d
//   p . v_hat(d) = sum_t p_t * (code_td * vs_t,g(d) + vz_t,g(d))
// Work split: the context is cut into units (a quantised chunk of G tokens, or
// up to 64 residual tokens); a workgroup takes a contiguous range of units
// (split-K), each of its 4 waves keeps its own online-softmax state over its
// units, the waves merge through LDS, and a second kernel merges the splits
// with log-sum-exp weights when there is more than one.  Scores are kept in the
// log2 domain (q is pre-scaled by scale * log2(e)) so exp is a single v_exp_f32.
#include <math.h>

#include <mutex>

#include "kivi_attention.hpp"
#include "kivi_common.hpp"
#include "../../include/kivi_hip.h"

namespace kivi {
namespace {

constexpr int kAttnWaves = 4;
constexpr int kAttnBlock = kAttnWaves * kWave;
constexpr int kMaxD = 256;
constexpr int kMaxSplits = 4096;       // the merge kernel keeps 2 floats per split in LDS
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const float* q;
    const uint8_t* k_codes;
    const float* k_scale;
    const float* k_zero;
    const uint8_t* v_codes;
    const float* v_scale;
    const float* v_zero;
    const void* k_res;  // ring of element type res_dt
    const void* v_res;
    float* out;
    float* part_o;     // [B, Hq, S, D]
    float* part_ml;    // [B, Hq, S, 2]
    int Hq, Hkv, D, G, Gv, Cmax, n_chunks, Rcap, res_start, res_len;
    int n_units, n_splits, units_per_split;
    float qscale;      // softmax scale * log2(e)
    int res_dt;        // 0 fp32, 1 bf16, 2 fp16
    QueryRows qr;      // HG query rows per kv head (kivi_attention.hpp)
    const int32_t* kv_start;   // [B] first visible position, or nullptr
    const uint32_t* hidden;    // per-sequence hidden-position bits (AttnLaunch), or nullptr
    int64_t hidden_stride;
};

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}

// lane l's value of v, for every lane (l wave-uniform)
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ int ring_slot(int start, int t, int cap) {
    int s = start + t;
    return s >= cap ? s - cap : s;
}

template <int HG>
__global__ __launch_bounds__(kAttnBlock) void attn_generic_kernel(AttnArgs a) {
    extern __shared__ float smem[];
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
    const int D = a.D, G = a.G;
    const int wave_floats = HG * D + HG * kWave;
    float* sq = smem;                                      // [HG][D]
    float* sqs = smem + HG * D + wave * wave_floats;       // [HG][D]  q * k_scale
    float* sp = sqs + HG * D;                              // [HG][64] probabilities
    const int64_t bh = (int64_t)b * a.Hkv + kvh;
    // left padding: context positions before kv_lo take no weight
    const int kv_lo = a.kv_start ? a.kv_start[b] : 0;
    // any other padding pattern: the sequence's hidden-position bits
    const uint32_t* hid_row = a.hidden ? a.hidden + b * a.hidden_stride : nullptr;

    for (int e = threadIdx.x; e < HG * D; e += kAttnBlock) {
        const int h = e / D, d = e % D;
        sq[e] = a.qr.real(h) ? a.q[a.qr.row(b, kvh, h, a.Hq, D) + d] * a.qscale : 0.f;
    }
    __syncthreads();

    float m[HG], l[HG], o[HG][kMaxD / kWave];
#pragma unroll
    for (int h = 0; h < HG; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxD / kWave; ++j) o[h][j] = 0.f;
    }

    const int u_begin = split * a.units_per_split;
    const int u_end = min(u_begin + a.units_per_split, a.n_units);
    for (int u = u_begin + wave; u < u_end; u += kAttnWaves) {
        float s[HG];
        bool valid;
        const bool quant = u < a.n_chunks;
        const int64_t cid = bh * a.Cmax + u;
        int rbase = 0, rcount = 0;
        if (quant) {
            // q * k_scale for this chunk, and the zero-point term per head.
            float bpart[HG];
#pragma unroll
            for (int h = 0; h < HG; ++h) bpart[h] = 0.f;
            for (int d = lane; d < D; d += kWave) {
                const float ks = a.k_scale[cid * D + d], kz = a.k_zero[cid * D + d];
#pragma unroll
                for (int h = 0; h < HG; ++h) {
                    const float qv = sq[h * D + d];
                    sqs[h * D + d] = qv * ks;
                    bpart[h] = fmaf(qv, kz, bpart[h]);
                }
            }
            float bias[HG];
#pragma unroll
            for (int h = 0; h < HG; ++h) bias[h] = wave_sum(bpart[h]);
            wave_sync();
            const int t = lane;
            valid = t < G && u * G + t >= kv_lo &&
                    !(hid_row && position_hidden(hid_row, u * G + t));
            float acc[HG];
#pragma unroll
            for (int h = 0; h < HG; ++h) acc[h] = 0.f;
            if (valid) {
                const uint32_t* kc =
                    reinterpret_cast<const uint32_t*>(a.k_codes + (cid * G + t) * (D / 4));
                for (int w4 = 0; w4 < D / 16; ++w4) {
                    const uint32_t w = kc[w4];
                    // dword w4 holds channels 16*w4 .. 16*w4+15; byte j bits 2k
                    // hold channel 16*w4 + 4j + k.
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t mk = (w >> (2 * k)) & 0x03030303u;
                        const float c0 = (float)(mk & 0xff), c1 = (float)((mk >> 8) & 0xff);
                        const float c2 = (float)((mk >> 16) & 0xff), c3 = (float)(mk >> 24);
                        const int ch = 16 * w4 + k;
#pragma unroll
                        for (int h = 0; h < HG; ++h) {
                            const float* qs = sqs + h * D + ch;
                            acc[h] = fmaf(qs[0], c0, acc[h]);
                            acc[h] = fmaf(qs[4], c1, acc[h]);
                            acc[h] = fmaf(qs[8], c2, acc[h]);
                            acc[h] = fmaf(qs[12], c3, acc[h]);
                        }
                    }
                }
            }
#pragma unroll
            for (int h = 0; h < HG; ++h) s[h] = valid ? acc[h] + bias[h] : -INFINITY;
        } else {
            rbase = (u - a.n_chunks) * kWave;
            rcount = min(kWave, a.res_len - rbase);
            const int t = rbase + lane;
            valid = lane < rcount && a.n_chunks * G + t >= kv_lo &&
                    !(hid_row && position_hidden(hid_row, a.n_chunks * G + t));
            float acc[HG];
#pragma unroll
            for (int h = 0; h < HG; ++h) acc[h] = 0.f;
            if (valid) {
                const int64_t kr = ((int64_t)bh * a.Rcap + ring_slot(a.res_start, t, a.Rcap)) * D;
                for (int d4 = 0; d4 < D / 4; ++d4) {
                    const float4 kv = load4_dt(a.k_res, kr + 4 * d4, a.res_dt);
#pragma unroll
                    for (int h = 0; h < HG; ++h) {
                        const float* qh = sq + h * D + 4 * d4;
                        acc[h] = fmaf(qh[0], kv.x, acc[h]);
                        acc[h] = fmaf(qh[1], kv.y, acc[h]);
                        acc[h] = fmaf(qh[2], kv.z, acc[h]);
                        acc[h] = fmaf(qh[3], kv.w, acc[h]);
                    }
                }
            }
            // row h sees the window's first qr.visible(h) tokens
#pragma unroll
            for (int h = 0; h < HG; ++h)
                s[h] = valid && t < a.qr.visible(h, a.res_len) ? acc[h] : -INFINITY;
        }

        // Online softmax (log2 domain).
#pragma unroll
        for (int h = 0; h < HG; ++h) {
            const float mnew = fmaxf(m[h], wave_max(s[h]));
            // a row may see no token of a residual unit (then m and mnew
            // can both be -inf): no weight, no rescale
            const float alpha = m[h] == -INFINITY ? 0.f : exp2f(m[h] - mnew);
            const float p = s[h] == -INFINITY ? 0.f : exp2f(s[h] - mnew);
            l[h] = l[h] * alpha + wave_sum(p);
            m[h] = mnew;
#pragma unroll
            for (int j = 0; j < kMaxD / kWave; ++j) o[h][j] *= alpha;
            sp[h * kWave + lane] = p;
        }
        wave_sync();

        if (quant) {
            const int gpt = D / a.Gv;
#pragma unroll
            for (int j = 0; j < kMaxD / kWave; ++j) {
                const int d = lane + kWave * j;
                if (d >= D) break;
                const int gd = d / a.Gv;
                const uint32_t* vc =
                    reinterpret_cast<const uint32_t*>(a.v_codes + (cid * D + d) * (G / 4));
                const float* vs = a.v_scale + (cid * gpt + gd) * G;   // [D/Gv][G]
                const float* vz = a.v_zero + (cid * gpt + gd) * G;
                for (int w4 = 0; w4 < G / 16; ++w4) {
                    const uint32_t w = vc[w4];
#pragma unroll
                    for (int byte = 0; byte < 4; ++byte) {
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const int tok = 16 * w4 + 4 * byte + k;
                            const uint32_t c = (w >> (8 * byte + 2 * k)) & 3u;
                            const float vh = decode1(c, vs[tok], vz[tok]);
#pragma unroll
                            for (int h = 0; h < HG; ++h)
                                o[h][j] = fmaf(sp[h * kWave + tok], vh, o[h][j]);
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < kMaxD / kWave; ++j) {
                const int d = lane + kWave * j;
                if (d >= D) break;
                for (int tt = 0; tt < rcount; ++tt) {
                    const float vv = load1_dt(
                        a.v_res,
                        ((int64_t)bh * a.Rcap + ring_slot(a.res_start, rbase + tt, a.Rcap)) * D + d,
                        a.res_dt);
#pragma unroll
                    for (int h = 0; h < HG; ++h)
                        o[h][j] = fmaf(sp[h * kWave + tt], vv, o[h][j]);
                }
            }
        }
        wave_sync();
    }

    // ---- merge the waves' states through LDS -------------------------------
    __syncthreads();
    float* mine = smem + HG * D + wave * wave_floats;      // [HG][D] o, then [HG] m, [HG] l
#pragma unroll
    for (int h = 0; h < HG; ++h) {
#pragma unroll
        for (int j = 0; j < kMaxD / kWave; ++j) {
            const int d = lane + kWave * j;
            if (d < D) mine[h * D + d] = o[h][j];
        }
        if (lane == 0) {
            mine[HG * D + h] = m[h];
            mine[HG * D + HG + h] = l[h];
        }
    }
    __syncthreads();
    const int64_t prow0 = ((int64_t)b * a.Hkv + kvh) * HG;      // partial rows
    for (int e = threadIdx.x; e < HG * D; e += kAttnBlock) {
        const int h = e / D, d = e % D;
        float M = -INFINITY;
        for (int w = 0; w < kAttnWaves; ++w)
            M = fmaxf(M, smem[HG * D + w * wave_floats + HG * D + h]);
        float acc = 0.f, L = 0.f;
        for (int w = 0; w < kAttnWaves; ++w) {
            const float* reg = smem + HG * D + w * wave_floats;
            const float mw = reg[HG * D + h];
            const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
            acc = fmaf(f, reg[h * D + d], acc);
            L = fmaf(f, reg[HG * D + HG + h], L);
        }
        if (!a.qr.real(h)) continue;     // a padding row
        if (a.n_splits == 1) {
            // (a row with no visible position -- every one hidden -- gives 0)
            a.out[a.qr.row(b, kvh, h, a.Hq, D) + d] = L > 0.f ? acc / L : 0.f;
        } else {
            const int64_t row = (prow0 + h) * a.n_splits + split;
            a.part_o[row * D + d] = acc;
            if (d == 0) {
                a.part_ml[row * 2] = M;
                a.part_ml[row * 2 + 1] = L;
            }
        }
    }
}

// Merge split partials: grid (Hkv * HG, B), one block per partial row
// (b, kv head, query row v), one thread per channel rounded up to whole
// waves (lanes past D take part in the reductions with -inf and store
// nothing; a partial wave would feed its inactive lanes' zeros into the
// shuffles), dynamic LDS of 2*S floats.  The S (m, l) pairs are read in parallel (one per thread) and
// turned into weights f_s = 2^(m_s - M) in LDS; each thread then sums its
// channel over the S partial rows with every load in flight at once (the
// loop is unrolled), so the kernel costs about two memory round trips
// however many splits there are.  The sums run in split order with fmaf, as
// a plain sequential merge would.
__global__ __launch_bounds__(kMaxD) void attn_merge_kernel(const float* __restrict__ part_o,
                                                           const float* __restrict__ part_ml,
                                                           float* __restrict__ out, QueryRows qr,
                                                           int Hq, int HG, int D, int S) {
    extern __shared__ float wl[];                 // [S] weights, then [S] l
    __shared__ float red[kMaxD / kWave];
    const int kvh = blockIdx.x / HG, v = blockIdx.x % HG;
    if (!qr.real(v)) return;                      // a padding row
    const int64_t row = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    float* const orow = out + qr.row(blockIdx.y, kvh, v, Hq, D);
    const float* ml = part_ml + row * S * 2;
    const int tid = threadIdx.x, nt = blockDim.x;
    float mloc = -INFINITY;
    for (int s = tid; s < S; s += nt) {
        const float m = ml[2 * s];
        wl[s] = m;
        wl[S + s] = ml[2 * s + 1];
        mloc = fmaxf(mloc, m);
    }
    mloc = wave_max(mloc);
    if (tid % kWave == 0) red[tid / kWave] = mloc;
    __syncthreads();
    float M = red[0];
    for (int w = 1; w < (nt + kWave - 1) / kWave; ++w) M = fmaxf(M, red[w]);
    for (int s = tid; s < S; s += nt) {
        const float m = wl[s];
        wl[s] = m == -INFINITY ? 0.f : exp2f(m - M);
    }
    __syncthreads();
    for (int d = tid; d < D; d += nt) {
        const float* po = part_o + row * S * D + d;
        float acc = 0.f, L = 0.f;
        int s = 0;
        for (; s + 8 <= S; s += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = po[(int64_t)(s + j) * D];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc = fmaf(wl[s + j], v[j], acc);
                L = fmaf(wl[s + j], wl[S + s + j], L);
            }
        }
        for (; s < S; ++s) {
            acc = fmaf(wl[s], po[(int64_t)s * D], acc);
            L = fmaf(wl[s], wl[S + s], L);
        }
        orow[d] = L > 0.f ? acc / L : 0.f;      // 0: every position hidden
    }
}

// The same merge for at most SM <= 64 splits in one memory round trip:
// each thread loads its channel's S partial outputs while lane s of each wave
// loads the row's pair (m_s, l_s); each wave then forms the maximum and the
// weights f_s = 2^(m_s - M) across its lanes and reads them back one split
// at a time (readlane): no LDS, no barrier between two dependent rounds.
// The operations and their order are attn_merge_kernel's (the fmaf sums run
// in split order), so the output bits are the same.  Threads past D load
// channel D-1 and store nothing.
template <int SM>
__global__ __launch_bounds__(kMaxD) void attn_merge_regs_kernel(const float* __restrict__ part_o,
                                                                const float* __restrict__ part_ml,
                                                                float* __restrict__ out,
                                                                QueryRows qr, int Hq, int HG,
                                                                int D, int S) {
    static_assert(SM <= kWave, "one split per lane");
    const int kvh = blockIdx.x / HG, v = blockIdx.x % HG;
    if (!qr.real(v)) return;                      // a padding row
    const int64_t row = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    const int lane = threadIdx.x % kWave;
    const float* ml = part_ml + row * S * 2 + 2 * min(lane, S - 1);
    const float m_s = ml[0], l_s = ml[1];
    const int d = min((int)threadIdx.x, D - 1);
    const float* po = part_o + row * S * D + d;
    float o[SM];
#pragma unroll
    for (int s = 0; s < SM; ++s) o[s] = po[(int64_t)min(s, S - 1) * D];
    const float M = wave_max(lane < S ? m_s : -INFINITY);
    const float f_s = lane < S && m_s != -INFINITY ? exp2f(m_s - M) : 0.f;
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int s = 0; s < SM; ++s) {
        if (s < S) {
            const float w = lane_f(f_s, s);
            acc = fmaf(w, o[s], acc);
            L = fmaf(w, lane_f(l_s, s), L);
        }
    }
    if ((int)threadIdx.x < D)        // 0: every position hidden
        out[qr.row(blockIdx.y, kvh, v, Hq, D) + d] = L > 0.f ? acc / L : 0.f;
}

struct Plan {
    int layout;
    bool mfma;                                // matrix-core kernel (else the generic one)
    int n_units, n_splits, units_per_split;   // generic kernel
    int n_qsplits, chunks_per_wave, res_waves, early_per_pass_x2;   // matrix-core kernel
};

// empty_ok: the caller can give the matrix-core kernel a readable chunk 0
// (non-null chunk arrays with capacity for one chunk) when the context has
// no chunk yet.
Plan make_plan(int B, int Hkv, int D, int G, int Gv, int n_chunks, int res_len,
               int splits_hint, bool empty_ok = true) {
    Plan p{};
    p.layout = code_layout_for(D, G, Gv);
    if (p.layout == kLayoutMfma && n_chunks == 0) {
        // A context still wholly in the residual window (the first steps of
        // every sequence).  The matrix-core kernel's window pass takes it: one
        // split, all four waves on the window; the prefetch ring's loads read
        // chunk 0 and go unused.  Without a readable chunk 0 the generic
        // kernel takes it, also unsplit, so that the workspace (none) does
        // not depend on which.  B=1 and 16, 32/8 heads, 100-127 tokens: 32-43
        // us per call on the generic kernel.
        p.mfma = empty_ok;
        p.n_units = (res_len + kWave - 1) / kWave;
        p.units_per_split = p.n_units;
        p.n_qsplits = p.n_splits = 1;
        p.chunks_per_wave = 0;
        p.res_waves = 4;
        p.early_per_pass_x2 = 0;
        return p;
    }
    p.mfma = p.layout == kLayoutMfma;
    if (p.mfma) {
        // Head_dim 128 (two workgroups per CU): the larger of two split
        // counts, then at least 2 chunks per wave:
        // (a) the most splits whose workgroups still fit the chip at once
        //     (512: two per CU) while every wave keeps >= 16 chunks, so that
        //     one wave per workgroup takes the residual window alone;
        // (b) enough splits for 256 workgroups (one per CU).
        // Swept over B = 1-64 sequences at 2K-32K contexts (32/8 heads, the
        // best split count per shape against this rule's): B=12 at 8K takes
        // 4 splits (31.5 us; the 2048-wave target below took 6: 39.6 us, 576
        // workgroups, the last 64 in a second round), B=24 2 (50.2 against
        // 60.0 us), B=8 4 (24.4 against 27.3 us), B=2 16 (17.3 against
        // 19.0 us); one sequence keeps 32, and configs 3, 4 and 5 keep 1, 1
        // and 16.
        // Other head dims aim for ~2048 chunk waves in flight with >= 2
        // chunks per wave: at head_dim 64 (three workgroups per CU, half the
        // bytes per chunk) that stayed ahead (B=16 and 4, 12/12 heads, 8K:
        // 28.0 and 15.2 us against 31.0 and 16.7 us with the rule above).
        constexpr int kWavesPerGroup = 4, kMinChunksPerWave = 2;
        constexpr int kSlots = 512, kCUs = 256;        // MI355X: 256 CUs, two workgroups each
        constexpr int kMinChunksForOneResWave = 16, kTargetWaves = 2048;
        int S = splits_hint;
        if (S <= 0) {
            const int pairs = B * Hkv;
            if (D == 128) {
                int sa = 1;
                for (int s = 2; s <= kMaxSplits && (int64_t)pairs * s <= kSlots; ++s)
                    if ((n_chunks + kWavesPerGroup * s - 1) / (kWavesPerGroup * s) >=
                        kMinChunksForOneResWave)
                        sa = s;
                S = max(max(sa, kCUs / pairs), 1);
            } else {
                S = (kTargetWaves + kWavesPerGroup * pairs - 1) / (kWavesPerGroup * pairs);
            }
            const int cap = (n_chunks + kWavesPerGroup * kMinChunksPerWave - 1) /
                            (kWavesPerGroup * kMinChunksPerWave);
            S = min(S, max(cap, 1));
        }
        // The residual window is taken in whole 16-token passes.  With
        // enough chunks per wave, the last wave of each workgroup takes all of
        // its split's passes while the other three start on chunks, taking
        // 3 chunks each per pass up front (measured best at config 4; the
        // launch doubles it for 8 query rows per kv head, whose passes cost
        // twice the score work); otherwise every wave takes passes before
        // its chunks.
        // every split gets at least one chunk
        S = max(1, min(min(S, kMaxSplits), (n_chunks + kWavesPerGroup - 1) / kWavesPerGroup));
        p.chunks_per_wave = (n_chunks + kWavesPerGroup * S - 1) / (kWavesPerGroup * S);
        p.n_qsplits = (n_chunks + kWavesPerGroup * p.chunks_per_wave - 1) /
                      (kWavesPerGroup * p.chunks_per_wave);
        constexpr int kEarlyPerPassX2 = 6;        // 3 chunk steps per residual pass
        if (res_len > 0 && p.chunks_per_wave >= kMinChunksForOneResWave) {
            p.res_waves = 1;
            p.early_per_pass_x2 = kEarlyPerPassX2;
        } else {
            p.res_waves = kWavesPerGroup;
            p.early_per_pass_x2 = 0;
        }
        p.n_splits = p.n_qsplits;
        return p;
    }
    p.n_units = n_chunks + (res_len + kWave - 1) / kWave;
    int S = splits_hint;
    if (S <= 0) {
        const int target_groups = 2048;
        S = (target_groups + B * Hkv - 1) / (B * Hkv);
    }
    S = max(1, min(min(S, kMaxSplits), (p.n_units + kAttnWaves - 1) / kAttnWaves));
    p.units_per_split = (p.n_units + S - 1) / S;
    p.n_splits = (p.n_units + p.units_per_split - 1) / p.units_per_split;
    return p;
}

// Partials (and the merge kernel) are needed whenever more than one
// workgroup covers a row.
bool needs_workspace(const Plan& p) { return p.n_splits > 1; }

// LDS per workgroup the current device allows (160 KB on gfx950).
int max_lds_bytes() {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) ==
            hipSuccess && v > 0)
        return v;
    return 160 * 1024;
}

// Rows per kv head of one launch: qlen * hg rounded up to a power of two.
int rows_for(int n) { return n <= 1 ? 1 : n <= 2 ? 2 : n <= 4 ? 4 : 8; }

// Widest rows per kv head of one launch: 8 (the kernels' widest instance),
// except on the matrix-core kernel at head_dim 256 with G = 64 and a run-time
// value-group count (group_size_v 64 or 128), whose 8-row instance needs more
// registers than a wave has (it spilled 264 bytes per lane): launches there
// take 4 rows.
int max_rows(bool mfma, int D, int G, int Gv) {
    return (mfma && D == 256 && G == 64 && Gv != 32 && Gv != D) ? 4 : 8;
}

// Query heads per kv head that one launch covers: all of them up to
// max_rows; more (multi-query models) take one launch per group of that
// many, each streaming the store once.
int heads_per_launch(int hg, int max_r) { return hg < max_r ? hg : max_r; }

// Head and group geometry every decode launch needs, whatever its context.
int check_geometry(int q_heads, int kv_heads, int head_dim, int group_size_k,
                   int group_size_v) {
    if (kv_heads <= 0 || q_heads <= 0 || q_heads % kv_heads)
        return set_error(kErrInvalidArgument,
                         "q_heads (%d) must be a positive multiple of kv_heads (%d)",
                         q_heads, kv_heads);
    if (head_dim <= 0 || head_dim % 16 || head_dim > kMaxD)
        return set_error(kErrUnsupported, "head_dim %d (supported: multiple of 16, <= %d)",
                         head_dim, kMaxD);
    if (group_size_k <= 0 || group_size_k % 4 || group_size_v <= 0 || group_size_v % 4 ||
        head_dim % group_size_v)
        return set_error(kErrInvalidArgument,
                         "group sizes must be positive multiples of 4 and group_size_v must "
                         "divide head_dim (got %d, %d, head_dim %d)", group_size_k,
                         group_size_v, head_dim);
    return kOk;
}

}  // namespace

int launch_attention_mfma(const AttnLaunch& a, hipStream_t st) {
    // every workgroup's prefetch ring reads at least one real chunk, or, in a
    // context with none yet, chunk 0 of a store that has room for one (one
    // split, its loads unused)
    const bool empty = a.n_chunks == 0 && a.n_qsplits == 1 && a.Cmax >= 1 && a.res_len > 0;
    if (!empty && (a.n_chunks <= 0 || a.chunks_per_wave <= 0 ||
                   (int64_t)(a.n_qsplits - 1) * 4 * a.chunks_per_wave >= a.n_chunks))
        return set_error(kErrInvalidArgument,
                         "matrix-core attention needs a chunk in every split (chunks %d, "
                         "splits %d, chunks per wave %d)", a.n_chunks, a.n_qsplits,
                         a.chunks_per_wave);
    const bool r16 = a.res_dt != kSrcF32;
    switch (a.qr.rows) {
        case 1: return r16 ? launch_attention_mfma_hg1_r16(a, st) : launch_attention_mfma_hg1(a, st);
        case 2: return r16 ? launch_attention_mfma_hg2_r16(a, st) : launch_attention_mfma_hg2(a, st);
        case 4: return r16 ? launch_attention_mfma_hg4_r16(a, st) : launch_attention_mfma_hg4(a, st);
        default: return r16 ? launch_attention_mfma_hg8_r16(a, st) : launch_attention_mfma_hg8(a, st);
    }
}
}  // namespace kivi

// Split partials of the allocation-free entry point: one copy of this array
// per GPU, held until the process ends.  Host code never passes `scratch`
// itself (in host code its name is a host-side stand-in, not a device
// address); it resolves the device address once per device and uses that.
static __device__ __align__(256) unsigned char scratch[KIVI_NOALLOC_SCRATCH_BYTES];

namespace kivi {
namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// The device address of `scratch` on the current device, resolved with
// hipGetSymbolAddress on the first call made with that device current.
int scratch_for_current_device(void** out) {
    int dev = -1;
    int rc = check_hip(hipGetDevice(&dev), "hipGetDevice");
    if (rc) return rc;
    if (dev < 0 || dev >= kMaxScratchDevices)
        return set_error(kErrUnsupported, "device %d: the allocation-free entry point supports "
                         "devices 0..%d", dev, kMaxScratchDevices - 1);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                       "hipGetSymbolAddress(scratch)");
        if (rc) return rc;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return kOk;
}

}  // namespace
}  // namespace kivi

using namespace kivi;

extern "C" {

int kivi_packed_decode_attention_supported(int32_t q_heads, int32_t kv_heads,
                                           int32_t head_dim, int32_t group_size_k,
                                           int32_t group_size_v) {
    int rc = check_geometry(q_heads, kv_heads, head_dim, group_size_k, group_size_v);
    if (rc) return rc;
    if (code_layout_for(head_dim, group_size_k, group_size_v) == kLayoutPlain) {
        if (group_size_k % 16 || group_size_k > kWave)
            return set_error(kErrUnsupported,
                             "group_size_k %d (supported: multiple of 16, <= 64)", group_size_k);
        return kOk;
    }
    const int mr = max_rows(true, head_dim, group_size_k, group_size_v);
    const int lds = attention_mfma_lds_bytes(rows_for(heads_per_launch(q_heads / kv_heads, mr)),
                                             head_dim, group_size_k, head_dim / group_size_v);
    const int limit = max_lds_bytes();
    if (lds < 0 || lds > limit)
        return set_error(kErrUnsupported,
                         "decode attention with q_heads/kv_heads=%d, head_dim=%d, G=%d, "
                         "group_size_v=%d needs %d bytes of LDS per workgroup; the device "
                         "allows %d", q_heads / kv_heads, head_dim, group_size_k,
                         group_size_v, lds, limit);
    return kOk;
}

}  // extern "C"

namespace {

// Query tokens per launch: as many as fill at most max_rows rows per kv head
// and, on the matrix-core kernel, fit its LDS.
int tokens_per_launch(int hg, int q_len, bool mfma, int D, int G, int Gv) {
    int t = max(1, min(max_rows(mfma, D, G, Gv) / hg, q_len));
    if (mfma) {
        static const int limit = max_lds_bytes();
        while (t > 1 && attention_mfma_lds_bytes(rows_for(t * hg), D, G, D / Gv) > limit) t /= 2;
    }
    return t;
}

size_t workspace_for(int batch, int q_len, int q_heads, int kv_heads, int head_dim,
                     int group_size_k, int group_size_v, int num_chunks, int res_len,
                     int num_splits) {
    if (batch <= 0 || kv_heads <= 0 || q_heads <= 0 || head_dim <= 0 || group_size_k <= 0 ||
        group_size_v <= 0 || q_len <= 0 || q_heads % kv_heads)
        return 0;
    const Plan p = make_plan(batch, kv_heads, head_dim, group_size_k, group_size_v, num_chunks,
                             res_len, num_splits);
    if (!needs_workspace(p)) return 0;
    const int hl = heads_per_launch(q_heads / kv_heads,
                                    max_rows(p.mfma, head_dim, group_size_k, group_size_v));
    const int rows = rows_for(
        tokens_per_launch(hl, q_len, p.mfma, head_dim, group_size_k, group_size_v) * hl);
    return (size_t)batch * kv_heads * rows * p.n_splits * (head_dim + 2) * sizeof(float);
}

// Attention of q_len query tokens per sequence (q [batch][q_len][q_heads]
// [head_dim], out likewise) over [packed history ; residual window]; causal:
// the queries are the window's last q_len tokens and token i sees the window
// up to itself, else every token sees the whole context.  Tokens are split
// across launches when q_len * (q_heads / kv_heads) exceeds 8 rows, and the
// query heads of a kv head in groups of 8 when there are more; each launch
// streams the store once.
int attention_impl(const float* q, int32_t q_len, int32_t causal, const int32_t* kv_start,
                   const uint32_t* hidden, int64_t hidden_stride, const uint8_t* k_codes,
                   const float* k_scale, const float* k_zero, const uint8_t* v_codes,
                   const float* v_scale, const float* v_zero, const void* k_res,
                   const void* v_res, int32_t res_dtype, float* out, void* workspace,
                   size_t workspace_bytes, int32_t batch, int32_t q_heads, int32_t kv_heads,
                   int32_t head_dim, int32_t group_size_k, int32_t group_size_v,
                   int32_t chunk_capacity, int32_t num_chunks, int32_t res_capacity,
                   int32_t res_start, int32_t res_len, float softmax_scale, int32_t num_splits,
                   const void* k_new, const void* v_new, int64_t new_sb, int64_t new_sh,
                   void* stream) {
    if (!q || !out)
        return set_error(kErrInvalidArgument, "null q/out pointer");
    if (batch <= 0)
        return set_error(kErrInvalidArgument, "batch %d must be positive", batch);
    int rc = check_geometry(q_heads, kv_heads, head_dim, group_size_k, group_size_v);
    if (rc) return rc;
    const int hg = q_heads / kv_heads;
    if (num_chunks < 0 || res_len < 0 || num_chunks + res_len == 0)
        return set_error(kErrInvalidArgument, "empty context (num_chunks=%d, res_len=%d)",
                         num_chunks, res_len);
    if (q_len < 1)
        return set_error(kErrInvalidArgument, "q_len %d must be positive", q_len);
    // One query token sees the whole context either way (a decode step whose
    // token was just flushed has res_len 0).
    if (causal && q_len > 1 && q_len > res_len)
        return set_error(kErrInvalidArgument,
                         "causal attention of %d query tokens needs them in the residual "
                         "window (res_len %d)", q_len, res_len);
    if (k_new && q_len != 1)
        return set_error(kErrInvalidArgument, "the fused append takes one query token");
    if (hidden) {
        const int64_t words = ((int64_t)num_chunks * group_size_k + res_len + 31) / 32;
        if ((uintptr_t)hidden % 4 || hidden_stride < words)
            return set_error(kErrInvalidArgument,
                             "hidden-position rows need %lld 4-byte-aligned words per sequence "
                             "(stride %lld)", (long long)words, (long long)hidden_stride);
    }
    const int layout = code_layout_for(head_dim, group_size_k, group_size_v);
    if (num_chunks > 0) {
        if (!k_codes || !k_scale || !k_zero || !v_codes || !v_scale || !v_zero)
            return set_error(kErrInvalidArgument, "null packed-store pointer");
        if (layout == kLayoutPlain && (group_size_k % 16 || group_size_k > kWave))
            return set_error(kErrUnsupported,
                             "group_size_k %d (supported: multiple of 16, <= 64)", group_size_k);
        if (num_chunks > chunk_capacity)
            return set_error(kErrInvalidArgument, "num_chunks %d exceeds capacity %d",
                             num_chunks, chunk_capacity);
    }
    if (res_dtype < kSrcF32 || res_dtype > kSrcF16)
        return set_error(kErrInvalidArgument, "res_dtype %d is not 0 (f32), 1 (bf16) or 2 (f16)",
                         res_dtype);
    if (res_len > 0) {
        if (!k_res || !v_res)
            return set_error(kErrInvalidArgument, "null residual pointer");
        if ((uintptr_t)k_res % 16 || (uintptr_t)v_res % 16)
            return set_error(kErrInvalidArgument, "residual ring must be 16-byte aligned");
        if (res_len > res_capacity || res_start < 0 || res_start >= res_capacity)
            return set_error(kErrInvalidArgument,
                             "residual window (start %d, len %d) outside capacity %d",
                             res_start, res_len, res_capacity);
    }
    const bool empty_ok = chunk_capacity >= 1 && k_codes && k_scale && k_zero && v_codes &&
                          v_scale && v_zero;
    const Plan p = make_plan(batch, kv_heads, head_dim, group_size_k, group_size_v, num_chunks,
                             res_len, num_splits, empty_ok);
    const int hl = heads_per_launch(hg, max_rows(p.mfma, head_dim, group_size_k, group_size_v));
    const int tpl = tokens_per_launch(hl, q_len, p.mfma, head_dim, group_size_k, group_size_v);
    const int rows = rows_for(tpl * hl);
    float* part_o = nullptr;
    float* part_ml = nullptr;
    if (needs_workspace(p)) {
        const size_t need = workspace_for(batch, q_len, q_heads, kv_heads, head_dim,
                                          group_size_k, group_size_v, num_chunks, res_len,
                                          num_splits);
        if (workspace == nullptr || workspace_bytes < need)
            return set_error(kErrInvalidArgument, "workspace of %zu bytes needed, got %zu",
                             need, workspace_bytes);
        part_o = (float*)workspace;
        part_ml = part_o + (size_t)batch * kv_heads * rows * p.n_splits * head_dim;
    }
    hipStream_t st = (hipStream_t)stream;
    const int new_slot = k_new ? (res_start + res_len - 1) % res_capacity : 0;
    if (k_new && !p.mfma) {
        // the generic kernel reads the ring only: file the token there first
        rc = kivi_store_append(k_new, v_new, res_dtype, new_sb, new_sh, 0, 1,
                               const_cast<void*>(k_res), const_cast<void*>(v_res), res_dtype,
                               batch, kv_heads, head_dim, res_capacity, new_slot, stream);
        if (rc) return rc;
    }
    const int64_t tok_stride = (int64_t)q_heads * head_dim;      // one query token
    // One launch per group of up to hl query heads of each kv head (h0) and
    // per group of query tokens that fills at most max_rows rows (i0).
    for (int h0 = 0; h0 < hg; h0 += hl)
    for (int i0 = 0; i0 < q_len; i0 += tpl) {
        QueryRows qr;
        qr.qlen = min(tpl, q_len - i0);
        qr.hg = min(hl, hg - h0);
        qr.hg_all = hg;
        qr.h0 = h0;
        for (int v = 0; v < qr.qlen * qr.hg; ++v) {
            qr.row_tok |= (uint32_t)(v / qr.hg) << (4 * v);
            qr.row_head |= (uint32_t)(v % qr.hg) << (4 * v);
        }
        qr.q_bstride = (int64_t)q_len * tok_stride;
        qr.vis0 = causal ? res_len - (q_len - 1 - i0) : res_len;
        qr.rows = rows;
        const float* qi = q + i0 * tok_stride;
        float* oi = out + i0 * tok_stride;
        if (p.mfma) {
            AttnLaunch L{qi, k_codes, k_scale, k_zero, v_codes, v_scale, v_zero, k_res, v_res,
                         oi, part_o, part_ml, batch, q_heads, kv_heads, head_dim, group_size_k,
                         group_size_v, chunk_capacity, num_chunks, res_capacity, res_start,
                         res_len, p.n_qsplits, p.chunks_per_wave, p.res_waves,
                         // 8 rows: 6 chunks per pass (B=64, 64/8 heads, 8K
                         // context: 134.2 -> 130.6 us; 5 and 7 per pass
                         // 132.4 and 132.6 us)
                         p.early_per_pass_x2 * (rows >= 8 ? 2 : 1), p.n_splits,
                         softmax_scale * kLog2e, k_new, v_new,
                         new_sb, new_sh, new_slot, res_dtype, qr, kv_start, hidden,
                         hidden_stride};
            rc = launch_attention_mfma(L, st);
        } else {
            AttnArgs a{qi, k_codes, k_scale, k_zero, v_codes, v_scale, v_zero, k_res, v_res, oi,
                       part_o, part_ml, q_heads, kv_heads, head_dim, group_size_k, group_size_v,
                       chunk_capacity, num_chunks, res_capacity, res_start, res_len, p.n_units,
                       p.n_splits, p.units_per_split, softmax_scale * kLog2e, res_dtype, qr,
                       kv_start, hidden, hidden_stride};
            const dim3 grid(p.n_splits, kv_heads, batch);
            const size_t lds = (size_t)(rows * head_dim +
                                        kAttnWaves * (rows * head_dim + rows * kWave)) *
                               sizeof(float);
            switch (rows) {
                case 1: attn_generic_kernel<1><<<grid, kAttnBlock, lds, st>>>(a); break;
                case 2: attn_generic_kernel<2><<<grid, kAttnBlock, lds, st>>>(a); break;
                case 4: attn_generic_kernel<4><<<grid, kAttnBlock, lds, st>>>(a); break;
                default: attn_generic_kernel<8><<<grid, kAttnBlock, lds, st>>>(a); break;
            }
            rc = check_launch("packed_attention");
        }
        if (rc) return rc;
        if (needs_workspace(p)) {
            // whole waves: the (m, l) reduction reads every lane of a wave
            const int merge_threads = (head_dim + kWave - 1) / kWave * kWave;
            const dim3 mgrid(kv_heads * rows, batch);
            const int S = p.n_splits;
            if (S <= 8)
                attn_merge_regs_kernel<8><<<mgrid, merge_threads, 0, st>>>(
                    part_o, part_ml, oi, qr, q_heads, rows, head_dim, S);
            else if (S <= 16)
                attn_merge_regs_kernel<16><<<mgrid, merge_threads, 0, st>>>(
                    part_o, part_ml, oi, qr, q_heads, rows, head_dim, S);
            else if (S <= 32)
                attn_merge_regs_kernel<32><<<mgrid, merge_threads, 0, st>>>(
                    part_o, part_ml, oi, qr, q_heads, rows, head_dim, S);
            else
                attn_merge_kernel<<<mgrid, merge_threads, 2 * S * sizeof(float), st>>>(
                    part_o, part_ml, oi, qr, q_heads, rows, head_dim, S);
            rc = check_launch("packed_attention_merge");
            if (rc) return rc;
        }
    }
    return kOk;
}

}  // namespace

extern "C" {

size_t kivi_packed_decode_attention_workspace_size(int32_t batch, int32_t q_heads,
                                                   int32_t kv_heads, int32_t head_dim,
                                                   int32_t group_size_k, int32_t group_size_v,
                                                   int32_t num_chunks, int32_t res_len,
                                                   int32_t num_splits) {
    return workspace_for(batch, 1, q_heads, kv_heads, head_dim, group_size_k, group_size_v,
                         num_chunks, res_len, num_splits);
}

size_t kivi_packed_attention_workspace_size(int32_t batch, int32_t q_len, int32_t q_heads,
                                            int32_t kv_heads, int32_t head_dim,
                                            int32_t group_size_k, int32_t group_size_v,
                                            int32_t num_chunks, int32_t res_len,
                                            int32_t num_splits) {
    return workspace_for(batch, q_len, q_heads, kv_heads, head_dim, group_size_k, group_size_v,
                         num_chunks, res_len, num_splits);
}

int kivi_packed_attention(const float* q, int32_t q_len, int32_t causal,
                          const int32_t* kv_start, const uint8_t* k_codes,
                          const float* k_scale, const float* k_zero, const uint8_t* v_codes,
                          const float* v_scale, const float* v_zero, const void* k_res,
                          const void* v_res, int32_t res_dtype, float* out, void* workspace,
                          size_t workspace_bytes, int32_t batch, int32_t q_heads,
                          int32_t kv_heads, int32_t head_dim, int32_t group_size_k,
                          int32_t group_size_v, int32_t chunk_capacity, int32_t num_chunks,
                          int32_t res_capacity, int32_t res_start, int32_t res_len,
                          float softmax_scale, int32_t num_splits, void* stream) {
    return attention_impl(q, q_len, causal, kv_start, nullptr, 0, k_codes, k_scale, k_zero,
                          v_codes, v_scale, v_zero, k_res, v_res, res_dtype, out, workspace,
                          workspace_bytes, batch, q_heads, kv_heads, head_dim, group_size_k,
                          group_size_v, chunk_capacity, num_chunks, res_capacity, res_start,
                          res_len, softmax_scale, num_splits, nullptr, nullptr, 0, 0, stream);
}

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
                                 void* stream) {
    return attention_impl(q, q_len, causal, kv_start, hidden, hidden_stride, k_codes, k_scale,
                          k_zero, v_codes, v_scale, v_zero, k_res, v_res, res_dtype, out,
                          workspace, workspace_bytes, batch, q_heads, kv_heads, head_dim,
                          group_size_k, group_size_v, chunk_capacity, num_chunks, res_capacity,
                          res_start, res_len, softmax_scale, num_splits, nullptr, nullptr, 0, 0,
                          stream);
}

int kivi_packed_decode_attention(const float* q, const uint8_t* k_codes, const float* k_scale,
                                 const float* k_zero, const uint8_t* v_codes,
                                 const float* v_scale, const float* v_zero, const void* k_res,
                                 const void* v_res, int32_t res_dtype, float* out, void* workspace,
                                 size_t workspace_bytes, int32_t batch, int32_t q_heads,
                                 int32_t kv_heads, int32_t head_dim, int32_t group_size_k,
                                 int32_t group_size_v, int32_t chunk_capacity,
                                 int32_t num_chunks, int32_t res_capacity, int32_t res_start,
                                 int32_t res_len, float softmax_scale, int32_t num_splits,
                                 void* stream) {
    return attention_impl(q, 1, 1, nullptr, nullptr, 0, k_codes, k_scale, k_zero, v_codes, v_scale,
                          v_zero, k_res, v_res, res_dtype, out, workspace, workspace_bytes, batch,
                          q_heads, kv_heads, head_dim, group_size_k, group_size_v, chunk_capacity,
                          num_chunks, res_capacity, res_start, res_len, softmax_scale, num_splits,
                          nullptr, nullptr, 0, 0, stream);
}

int kivi_packed_decode_attention_noalloc(
        const float* q, const uint8_t* k_codes, const float* k_scale, const float* k_zero,
        const uint8_t* v_codes, const float* v_scale, const float* v_zero, const void* k_res,
        const void* v_res, int32_t res_dtype, float* out, int32_t batch, int32_t q_heads,
        int32_t kv_heads, int32_t head_dim, int32_t group_size_k, int32_t group_size_v,
        int32_t chunk_capacity, int32_t num_chunks, int32_t res_capacity, int32_t res_start,
        int32_t res_len, float softmax_scale, int32_t num_splits, void* stream) {
    const size_t need = kivi_packed_decode_attention_workspace_size(
        batch, q_heads, kv_heads, head_dim, group_size_k, group_size_v, num_chunks, res_len,
        num_splits);
    if (need > (size_t)KIVI_NOALLOC_SCRATCH_BYTES)
        return set_error(kErrInvalidArgument,
                         "this launch needs %zu bytes of split partials; the allocation-free "
                         "entry point holds at most %zu (pass fewer splits, or use "
                         "kivi_packed_decode_attention with a workspace)", need,
                         (size_t)KIVI_NOALLOC_SCRATCH_BYTES);
    // The scratch address of this device is resolved on the first call made
    // with it current, and kept.
    void* ws = nullptr;
    const int rc = scratch_for_current_device(&ws);
    if (rc) return rc;
    return attention_impl(q, 1, 1, nullptr, nullptr, 0, k_codes, k_scale, k_zero, v_codes, v_scale,
                          v_zero, k_res, v_res, res_dtype, out, ws, KIVI_NOALLOC_SCRATCH_BYTES,
                          batch, q_heads, kv_heads, head_dim, group_size_k, group_size_v,
                          chunk_capacity, num_chunks, res_capacity, res_start, res_len,
                          softmax_scale, num_splits, nullptr, nullptr, 0, 0, stream);
}

int kivi_packed_decode_attention_append(
        const float* q, const void* k_new, const void* v_new, int64_t new_batch_stride,
        int64_t new_head_stride, const uint8_t* k_codes, const float* k_scale,
        const float* k_zero, const uint8_t* v_codes, const float* v_scale, const float* v_zero,
        void* k_res, void* v_res, int32_t res_dtype, float* out, void* workspace,
        size_t workspace_bytes,
        int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t head_dim,
        int32_t group_size_k, int32_t group_size_v, int32_t chunk_capacity, int32_t num_chunks,
        int32_t res_capacity, int32_t res_start, int32_t res_len, float softmax_scale,
        int32_t num_splits, void* stream) {
    if (!k_new || !v_new)
        return set_error(kErrInvalidArgument, "null new-token pointer");
    if (!k_res || !v_res || res_len < 1)
        return set_error(kErrInvalidArgument,
                         "the window must hold the new token (res_len %d >= 1)", res_len);
    if (res_dtype < kSrcF32 || res_dtype > kSrcF16)
        return set_error(kErrInvalidArgument, "res_dtype %d is not 0 (f32), 1 (bf16) or 2 (f16)",
                         res_dtype);
    // rows of the ring's type, four channels per aligned load
    const int64_t vb = 4 * src_size(res_dtype);
    if (new_batch_stride < 0 || new_head_stride < 0 ||
        (new_batch_stride * src_size(res_dtype)) % vb ||
        (new_head_stride * src_size(res_dtype)) % vb || (uintptr_t)k_new % vb ||
        (uintptr_t)v_new % vb)
        return set_error(kErrInvalidArgument,
                         "new-token rows must be %d-byte aligned (strides multiples of 4)",
                         (int)vb);
    return attention_impl(q, 1, 1, nullptr, nullptr, 0, k_codes, k_scale, k_zero, v_codes, v_scale,
                          v_zero, k_res, v_res, res_dtype, out, workspace, workspace_bytes, batch,
                          q_heads, kv_heads, head_dim, group_size_k, group_size_v, chunk_capacity,
                          num_chunks, res_capacity, res_start, res_len, softmax_scale, num_splits,
                          k_new, v_new, new_batch_stride, new_head_stride, stream);
}

}  // extern "C"
