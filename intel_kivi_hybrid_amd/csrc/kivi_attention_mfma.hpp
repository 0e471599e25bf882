// Fused packed-KV decode attention on the gfx950 matrix cores.
//
// No reference counterpart (the reference dequantises flushed chunks into an
// fp32 CPU history and runs HF attention over it, src/kivi_sycl/cache/
// manager.py:251-290; the math is stated in tests/integration/
// test_attention_fix.py:40-43).  For one query token per sequence and the
// Hq/Hkv = HG query heads that share a kv head:
//
//   s[h,t] = sum_d q[h,d] * k_hat[t,d],  k_hat[t,d] = c[t,d]*ks[d] + kz[d]
//   o[h,d] = sum_t softmax(s)[h,t] * v_hat[t,d],
//            v_hat[t,d] = c'[t,d]*vs[t,g(d)] + vz[t,g(d)]
//
// over the packed chunks of the store, and the same over the fp32 residual
// window.  Decode at GQA ratio HG needs ~4*HG multiply-adds per 2-bit code;
// at fp32 VALU rates that, not HBM, would bound the kernel, so the two
// contractions run as bf16 MFMAs (v_mfma_f32_16x16x32_bf16) with fp32
// accumulation:
//
// * B operands are the codes themselves, read in place.  The store keeps each
//   lane's codes in MFMA operand order (kLayoutMfma): the codes of operand
//   dword k sit at bits 2k..2k+1 of the low byte of each 16-bit half (tile
//   0; tile 1 one byte up).  A half holding nothing but c << 2k is the bf16
//   bit pattern of c * 2^(2k-133), exactly: bf16 patterns below 256 are the
//   integers 0..255 times 2^-133 (subnormals, continued by the first normal
//   binade).  So an operand dword is one AND of the code word (tile 1: of
//   the word shifted down a byte), and the matrix cores, which take
//   subnormal bf16 inputs exactly on gfx950, multiply by c itself.
// * A operands carry the fp32 factors split into bf16 pieces (hi + mid + lo,
//   ~2^-25 relative, or hi + lo, ~2^-17): the key A matrix holds
//   q[h,d]*ks[d], the value A matrix p[h,t]*vs[t,g], each scaled by
//   2^(133-2k-64) for its operand position k (kCodeScale), so that products
//   come out in units of 2^-64.  The scales are multiplied by those powers of
//   two once, when a chunk's metadata is staged.
// * The zeros fold into corrections that are linear in the data:
//     s[h,t] = sum_d (q ks)[h,d] c + sum_d q[h,d] kz[d]
//     o[h,d] = sum_t (p vs)[h,t] c' + sum_t p[h,t] vz[t]
//   The key correction is summed over each head's operand-build lanes with
//   DPP, which leaves it in the lanes holding that head's scores, and added
//   in fp32 as the scores are scaled back by 2^64; the value correction is
//   accumulated per lane and added to the output.
//   The units bound the factors: the key product q*ks*softmax_scale*log2(e)
//   and the key scale below 2^59, value scales below 2^51 (larger ones
//   overflow the A operand to inf).  Value codes' products below ~2^-38
//   lose relative precision (fp32 subnormals).
//
// Work split: each wave owns a contiguous range of chunks of one
// (batch, kv-head) and keeps an online softmax over it in the log2 domain
// (q is pre-scaled by softmax_scale * log2(e)).  The running maximum is only
// moved when a chunk exceeds it by more than 8 (probabilities stay <= 256),
// so rescaling the accumulators is rare.  Workgroups of 4 waves merge their
// states in LDS; workgroups past the chunk splits take the fp32 residual
// window (fp32, bf16 or fp16 elements, widened) with plain fp32 FMAs.  Each workgroup writes a partial (o, m, l)
// that kivi_attention.hip's merge kernel combines with log-sum-exp weights.
#pragma once

#include <math.h>

#include <type_traits>

#include "kivi_common.hpp"
#include "kivi_attention.hpp"

namespace kivi {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;

template <int V>
struct Int {
    static constexpr int value = V;
};

// f(Int<K>{}), ..., f(Int<N-1>{}): a loop whose index is a constant expression.
template <int K, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (K < N) {
        f(Int<K>{});
        static_for<K + 1, N>(f);
    }
}
constexpr int kBlock = kWaves * kWave;
constexpr int kResPass = 16;              // residual tokens per pass of a wave
constexpr float kRescaleThreshold = 8.0f;   // log2 units

// Orders a wave's LDS writes before its own later LDS reads (other lanes of
// the same wave read what a lane wrote).  A wave's LDS operations execute in
// program order, so no wait is needed for that: the fences are at wavefront
// scope, which keeps the compiler from moving LDS accesses across this point
// and emits no s_waitcnt.  (Workgroup scope made every such point wait for
// the wave's LDS writes to complete: 1.3 % slower at config 4.)  Never used
// for data passed between waves; that takes lds_barrier().
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    bf16x2_t v = {(__bf16)a, (__bf16)b};   // round to nearest even
    return __builtin_bit_cast(uint32_t, v);
}

// The bf16 pairs (-1, 0) and (0, -1), held in VGPRs: split_pair's v_dot2
// reads them as register operands.  (As literals, the compiler's encoding of
// the (-1, 0) pair made the instruction read the pair's high half -- measured
// on gfx950 -- so the values are hidden from it.)
struct SplitConsts {
    uint32_t neg_x, neg_y;
};
__device__ __forceinline__ SplitConsts split_consts() {
    SplitConsts c{0x0000bf80u, 0xbf800000u};
    asm("" : "+v"(c.neg_x));
    asm("" : "+v"(c.neg_y));
    return c;
}

// (a, b) -> hi and lo bf16 pairs with a ~ hi.x + lo.x, b ~ hi.y + lo.y.
// a - hi.x is exact in fp32 (hi.x is a rounded to 8 significant bits), so
// one v_dot2_f32_bf16 of hi with (-1, 0) accumulated onto a forms it: two
// ops instead of widening hi's halves and subtracting (bit-identical over
// 8.4 M random pairs on gfx950, tiny normals included).
__device__ __forceinline__ void split_pair(float a, float b, uint32_t& hi, uint32_t& lo,
                                           SplitConsts k) {
    hi = pack_bf16x2(a, b);
    const bf16x2_t h2 = __builtin_bit_cast(bf16x2_t, hi);
    const float la = __builtin_amdgcn_fdot2_f32_bf16(h2, __builtin_bit_cast(bf16x2_t, k.neg_x), a,
                                                     false);
    const float lb = __builtin_amdgcn_fdot2_f32_bf16(h2, __builtin_bit_cast(bf16x2_t, k.neg_y), b,
                                                     false);
    lo = pack_bf16x2(la, lb);
}

// Three pieces: a ~ hi.x + mid.x + lo.x, b likewise (~2^-25 relative).  Each
// residual is exact in fp32 (the piece taken off is the value rounded to 8
// significant bits), so only lo's rounding remains.
__device__ __forceinline__ void split3_pair(float a, float b, uint32_t& hi, uint32_t& mid,
                                            uint32_t& lo, SplitConsts k) {
    hi = pack_bf16x2(a, b);
    const bf16x2_t h2 = __builtin_bit_cast(bf16x2_t, hi);
    const float ra = __builtin_amdgcn_fdot2_f32_bf16(h2, __builtin_bit_cast(bf16x2_t, k.neg_x), a,
                                                     false);
    const float rb = __builtin_amdgcn_fdot2_f32_bf16(h2, __builtin_bit_cast(bf16x2_t, k.neg_y), b,
                                                     false);
    mid = pack_bf16x2(ra, rb);
    const bf16x2_t m2 = __builtin_bit_cast(bf16x2_t, mid);
    const float sa = __builtin_amdgcn_fdot2_f32_bf16(m2, __builtin_bit_cast(bf16x2_t, k.neg_x), ra,
                                                     false);
    const float sb = __builtin_amdgcn_fdot2_f32_bf16(m2, __builtin_bit_cast(bf16x2_t, k.neg_y), rb,
                                                     false);
    lo = pack_bf16x2(sa, sb);
}

// Code word -> B operand of tile M (four dwords of two bf16 each).  Element j
// of the tile sits at bit 8M + 2(j/2) of the low (j even) or high (j odd)
// half of the word; dword k keeps bits 2k..2k+1 of each half of the word
// (tile 1: shifted down 8 bits), i.e. the values c * 2^(2k-133).  Plain
// C++, no inline asm: the result feeds matrix-core operands, and the
// compiler must see the VALU write to insert the wait states a VALU-write ->
// MFMA-read dependency needs.  (The earlier form, 8 + c with c moved to
// mantissa bits 5:4, took a shift and an and-or per dword: 15 VALU per word
// against 9.)
template <int M>
__device__ __forceinline__ bf16x8_t unpack_codes(uint32_t x) {
    const uint32_t y = M == 0 ? x : x >> 8;
    const u32x4_t o = {y & 0x00030003u, y & 0x000c000cu, y & 0x00300030u, y & 0x00c000c0u};
    return __builtin_bit_cast(bf16x8_t, o);
}

// Units of the products: A factors at operand position k carry
// 2^(kCodeExp - 2k - kProdExp) (kCodeExp = 133 undoes the code operand's
// 2^(2k-133)), so every matrix-core product and accumulator is the true
// value times 2^-kProdExp.
constexpr int kCodeExp = 133;
constexpr int kProdExp = 64;
constexpr float kProdUnit = 0x1p-64f;      // 2^-kProdExp
constexpr float kProdScale = 0x1p64f;      // 2^kProdExp
static_assert(kCodeExp - kProdExp == 69, "code scale constants below");

__device__ __forceinline__ f32x4_t mfma(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Reductions across the 16 lanes of a DPP row (row_ror 8, 4, 2, 1).
__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp<0x128>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x122>(v));
    return fmaxf(v, dpp<0x121>(v));
}

__device__ __forceinline__ float row_sum16(float v) {
    v += dpp<0x128>(v);
    v += dpp<0x124>(v);
    v += dpp<0x122>(v);
    return v + dpp<0x121>(v);
}

// Across the wave: DPP within each 16-lane row, then the four row results
// through readlane.  (__shfl_xor compiles to ds_bpermute, a chain of six LDS
// round trips.)
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max16(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row_sum16(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// A per-lane LDS address, computed once and kept in a VGPR (PIN).  Left to
// itself the compiler rebuilds such addresses (a multiply and an add of the
// wave's base) at every use in the chunk loop; the empty asm hides the
// value.  The pointer stays an LDS pointer, so constant offsets added to it
// fold into the ds instructions' offset field.  Each pinned address holds a
// VGPR for the whole loop: instances without the registers to spare
// (Shape::PIN false) leave the addresses to the compiler.
template <bool PIN, class T>
__device__ __forceinline__ T* pin_lds(T* p) {
    if constexpr (!PIN) return p;
    typedef __attribute__((address_space(3))) T lds_t;
    lds_t* q = (lds_t*)p;
    asm("" : "+v"(q));
    return (T*)q;
}

// Item number of a lane for the value operand build (a permutation of 0..63).
__device__ __forceinline__ int item_lane(int lane) {
    const int r = lane & 31;
    int v;
    if (r < 4 || r >= 28) v = r;              // 0-3 -> 0-3, 28-31 -> 28-31
    else if (r < 12) v = r + 12;              // 4-11 -> 16-23
    else if (r < 16) v = r - 8;               // 12-15 -> 4-7
    else if (r < 20) v = r + 8;               // 16-19 -> 24-27
    else v = r - 12;                          // 20-27 -> 8-15
    return (lane & 32) | v;
}

// Compile-time shape of one instantiation.
template <int HG_, int D_, int G_>
struct Shape {
    static constexpr int HG = HG_, D = D_, G = G_;
    static constexpr int NSUB = G / 32;              // 32-token sub-chunks
    static constexpr int NP = G * D / 1024;          // code dwords per lane
    static constexpr int KS = D / 32;                // key k-steps
    static constexpr int NBV = D / 16;               // value n-blocks
    static constexpr int LPH = (64 / HG < D / 2) ? 64 / HG : D / 2;   // W-prep lanes per head
    static constexpr int CPL = D / LPH;              // channels per W-prep lane
    static constexpr int NGMAX = D / 32;             // value groups (Gv >= 32)
    // chunk metadata: ks [D], kz [D], vs [NG][G], vz [NG][G] as float4s
    static constexpr int META4_MAX = (2 * D + 2 * NGMAX * G) / 4;
    static constexpr int NMETA = (META4_MAX + 63) / 64;      // float4 loads per lane
    // chunks kept in flight per wave: ~64 VGPRs of prefetch ring, and at
    // least 2 (the pipelined loop holds chunks i and i+1 at once).  With 8
    // query heads per kv head the operand builds hold twice the products per
    // lane, and two waves per SIMD fit only with half the ring (32 VGPRs):
    // with 64/8 heads, head_dim 128, that measured 25-30 % faster than a
    // 4-deep ring at one wave per SIMD (B=4-64, 8K-32K context), and 7-12 %
    // faster than a 4-deep ring at two waves, which spills (the same at
    // B=64).
    static constexpr int REGS_PER_CHUNK = 2 * NP + 4 * NMETA;
    static constexpr int RING_REGS = HG >= 8 ? 32 : 64;
    static constexpr int PF = (RING_REGS / REGS_PER_CHUNK) < 2 ? 2
                              : (RING_REGS / REGS_PER_CHUNK) > 4 ? 4
                              : RING_REGS / REGS_PER_CHUNK;
    // Per-wave LDS (bytes).  gfx950 LDS serves a ds_read_b128 16 lanes per
    // cycle from 64 banks of 4 bytes, the lanes {0-3, 12-15, 20-27} then
    // {4-11, 16-19, 28-31} of each half-wave; a ds_write_b128 8 consecutive
    // lanes per cycle from 32 banks; b32 accesses 32 lanes from 32 banks.
    // An A-operand read takes row l%16 and k-group l/16: with rows 2 (mod 4)
    // 16-byte slots apart, each read cycle hits 16 distinct slots (mod 16).
    static constexpr int WA_ROW = D + 16;            // bf16 per key A row
    static constexpr int PA_ROW = G + 16;            // bf16 per value A row
    // Key A factors are split into KP bf16 pieces: hi + mid + lo (~2^-25
    // relative) with up to 4 query heads per kv head, hi + lo (~2^-17) with
    // 8, where the 16 A rows are all taken.  The scores' error grows with
    // their size: with codes entering as 8 + c (an earlier operand form,
    // whose correction cancelled the 8 and so amplified the factors' rounding
    // ~8x) and two pieces, the output error reached ~1e-3 at a largest score
    // of 64 (natural units) at config 4's shape and at head_dim 64.
    static constexpr int KP = HG <= 4 ? 3 : 2;
    // Keep loop addresses and the correction's B operand in VGPRs (pin_lds):
    // ~13 VALU per chunk fewer for ~11 VGPRs, which the 8-head instances
    // (at the 256-register limit of two waves per SIMD) do not have.
    static constexpr bool PIN = HG <= 4;
    static constexpr int KROWS = KP * HG;            // key A rows holding data
    // A operands have 16 rows, of which only KROWS (key) or 2*HG (value: hi
    // / lo per head) carry data: the rest are stored once, as one zero row
    // that those lanes read.
    static constexpr int KAROWS = KROWS < 16 ? KROWS + 1 : 16;
    static constexpr int AROWS = 2 * HG < 16 ? 2 * HG + 1 : 16;
    static constexpr int PA_MAT = AROWS * PA_ROW;    // bf16 per value A matrix (one group)
    static constexpr int PL_ROW = G + 8;             // floats per probability row
    static constexpr int OFF_WA = 0;
    static constexpr int OFF_PA = OFF_WA + KAROWS * WA_ROW * 2;
    // The rest depends on the number of value groups NG = D / Gv.
    __host__ __device__ static constexpr int off_pl(int NG) { return OFF_PA + NG * PA_MAT * 2; }
    __host__ __device__ static constexpr int off_al(int NG) { return off_pl(NG) + 2 * HG * PL_ROW * 4; }
    // The value corrections [HG][NG][G/8] fp32 are staged only between
    // whole rings and after the chunk loop, when the key A operands are dead
    // (every step's key operand build rewrites all KROWS data rows before its
    // scores read them), so they share the key A rows.  That keeps a
    // workgroup at 8 query heads per kv head (head_dim 128, G=32) within
    // 80 KB of LDS: two workgroups per CU instead of one.
    __host__ __device__ static constexpr int off_vb(int NG) { return OFF_WA; }
    __host__ __device__ static constexpr int off_mt(int NG) { return off_al(NG) + 2 * 16 * 4; }
    __host__ __device__ static constexpr int meta_floats(int NG) { return 2 * D + 2 * NG * G; }
    // Staged metadata is stored with one empty 16-byte slot after every 16
    // (float4 slot s at slot s + s/16): the key operand build reads float4s
    // 2 apart per lane, and the value operand build reads them 2 apart per
    // item, which then fall on 16 distinct slots (mod 16) per read cycle.
    __host__ __device__ static constexpr int meta_slot(int s) { return s + s / 16; }
    __host__ __device__ static constexpr int meta_stride(int NG) {     // floats per buffer
        return 4 * (meta_slot(meta_floats(NG) / 4 - 1) + 1);
    }
    __host__ __device__ static constexpr int wave_lds(int NG) {
        return off_mt(NG) + 2 * meta_stride(NG) * 4;
    }
    // merge region: one state (o [HG][D], m [HG], l [HG] fp32) per wave; it
    // overlaps the per-wave regions, which are free before and after the
    // chunk loop
    static constexpr int RSTATE = HG * D + 2 * HG;
    static constexpr int MERGE_LDS = kWaves * RSTATE * 4;
    // residual pass: scaled q [HG][D] and per-wave probabilities [HG][16].
    // They sit in the last wave's region, which that wave uses for chunks
    // only after its residual pass (the last wave takes the whole window when
    // one wave does), past the merge slots that the passes of all waves may
    // write.
    static constexpr int QRES_LDS = HG * D * 4 + kWaves * HG * kResPass * 4;
    __host__ __device__ static constexpr int qres_off(int NG) { return (kWaves - 1) * wave_lds(NG); }
    // the combined state of the workgroup's residual slices, kept to the end
    static constexpr int RES_LDS = RSTATE * 4;
    __host__ __device__ static constexpr int lds(int NG) {
        return (kWaves * wave_lds(NG) > MERGE_LDS ? kWaves * wave_lds(NG) : MERGE_LDS) + RES_LDS;
    }
    __host__ __device__ static constexpr int res_off(int NG) { return lds(NG) - RES_LDS; }
    static_assert(NP >= 1 && LPH * CPL == D && CPL % 2 == 0, "shape");
    // NG = 1 gives the smallest per-wave region
    static_assert(QRES_LDS <= wave_lds(1) && MERGE_LDS <= qres_off(1), "residual buffers");
    static_assert(HG * NGMAX * (G / 8) * 4 <= KROWS * WA_ROW * 2,
                  "value corrections fit in the key A data rows");
};

// Writes this wave's state (o unnormalised over D channels, m, l) to the
// merge region; `o_of(h, d)` supplies o.
__device__ __forceinline__ float* merge_slot(unsigned char* smem, int HG, int D, int wave) {
    return reinterpret_cast<float*>(smem) + wave * (HG * D + 2 * HG);
}

// Folds the 4 residual-slice states parked in the merge slots into one state
// at `rstate` (the merge slots are free again afterwards).
template <int HG, int D>
__device__ void combine_residual(unsigned char* smem, float* rstate) {
    __syncthreads();
    for (int e = threadIdx.x; e < HG * D; e += kBlock) {
        const int h = e / D, d = e % D;
        float M = -INFINITY;
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, merge_slot(smem, HG, D, w)[HG * D + h]);
        float acc = 0.f, L = 0.f;
        for (int w = 0; w < kWaves; ++w) {
            const float* s = merge_slot(smem, HG, D, w);
            const float mw = s[HG * D + h];
            const float f = mw == -INFINITY ? 0.f : exp2_fast(mw - M);
            acc = fmaf(f, s[h * D + d], acc);
            L = fmaf(f, s[HG * D + HG + h], L);
        }
        rstate[h * D + d] = acc;
        if (d == 0) {
            rstate[HG * D + h] = M;
            rstate[HG * D + HG + h] = L;
        }
    }
    __syncthreads();
}

// Combines the 4 chunk states (merge slots) and the combined residual state
// of the workgroup and writes one partial (o, m, l) row per query head, or the
// normalised output when the workgroup is the row's only split.
template <int HG, int D, bool MASK>
__device__ void merge_and_store(unsigned char* smem, const float* rstate, const AttnLaunch& a,
                                int split, int kvh, int b) {
    __syncthreads();
    const int64_t prow0 = ((int64_t)b * a.Hkv + kvh) * HG;     // partial rows
    for (int e = threadIdx.x; e < HG * D; e += kBlock) {
        const int h = e / D, d = e % D;
        float M = -INFINITY;
        for (int w = 0; w <= kWaves; ++w) {
            const float* s = w < kWaves ? merge_slot(smem, HG, D, w) : rstate;
            M = fmaxf(M, s[HG * D + h]);
        }
        float acc = 0.f, L = 0.f;
        for (int w = 0; w <= kWaves; ++w) {
            const float* s = w < kWaves ? merge_slot(smem, HG, D, w) : rstate;
            const float mw = s[HG * D + h];
            const float f = mw == -INFINITY ? 0.f : exp2_fast(mw - M);
            acc = fmaf(f, s[h * D + d], acc);
            L = fmaf(f, s[HG * D + HG + h], L);
        }
        if (!a.qr.real(h)) continue;    // a padding row
        if (a.n_splits == 1) {          // the only partial of its row: finish here
            if constexpr (MASK)         // a row with no visible position gives 0
                a.out[a.qr.row(b, kvh, h, a.Hq, D) + d] = L > 0.f ? acc / L : 0.f;
            else
                a.out[a.qr.row(b, kvh, h, a.Hq, D) + d] = acc / L;
            continue;
        }
        const int64_t row = (prow0 + h) * a.n_splits + split;
        a.part_o[row * D + d] = acc;
        if (d == 0) {
            a.part_ml[row * 2] = M;
            a.part_ml[row * 2 + 1] = L;
        }
    }
}

// ---------------------------------------------------------------------------
// Quantised chunks (matrix cores).
// ---------------------------------------------------------------------------
template <class S>
struct ChunkRegs {
    uint32_t kc[S::NP];      // this lane's key code words
    uint32_t vc[S::NP];      // this lane's value code words
    float4 meta[S::NMETA];   // slice of [ks | kz | vs | vz]
};

// Per-lane sources of a chunk's loads, computed once per wave: the lane's code
// words, and for each float4 of the metadata sweep [ks | kz | vs | vz] the
// address at chunk 0 of this (b, kv-head) and the per-chunk stride.
template <class S>
struct ChunkSrc {
    const uint32_t* kc;
    const uint32_t* vc;
    const float4* meta[S::NMETA];
    int meta_stride[S::NMETA];    // float4s per chunk
};

// Paired metadata sweep (PAIRED): the first NMETA/2 float4s of a lane are
// scales, from [ks | vs], and the last NMETA/2 the zeros of the same
// channels or tokens, from [kz | vz]: a lane's scale float4s are then known
// at compile time (they alone are multiplied when staged).  Used where it
// needs no more loads per lane than the plain sweep.
template <class S>
constexpr bool paired_meta(int NG) {
    return NG > 0 && 2 * ((S::D / 4 + NG * S::G / 4 + 63) / 64) <= S::NMETA && S::NMETA % 2 == 0;
}

template <class S, bool PAIRED>
__device__ __forceinline__ ChunkSrc<S> chunk_src(const AttnLaunch& a, int64_t cid0, int lane,
                                                 int NG) {
    ChunkSrc<S> c;
    c.kc = reinterpret_cast<const uint32_t*>(a.k_codes) + cid0 * (64 * S::NP) + lane * S::NP;
    c.vc = reinterpret_cast<const uint32_t*>(a.v_codes) + cid0 * (64 * S::NP) + lane * S::NP;
    const int kq = S::D / 4, vq = NG * S::G / 4;
    if constexpr (PAIRED) {
        constexpr int HALF = S::NMETA / 2;
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
            const int e = min(lane + 64 * i, kq + vq - 1);     // past the end: reload the last
            if (e < kq) {
                c.meta[i] = reinterpret_cast<const float4*>(a.k_scale + cid0 * S::D) + e;
                c.meta[i + HALF] = reinterpret_cast<const float4*>(a.k_zero + cid0 * S::D) + e;
                c.meta_stride[i] = c.meta_stride[i + HALF] = kq;
            } else {
                c.meta[i] = reinterpret_cast<const float4*>(a.v_scale + cid0 * NG * S::G) + (e - kq);
                c.meta[i + HALF] = reinterpret_cast<const float4*>(a.v_zero + cid0 * NG * S::G) +
                                   (e - kq);
                c.meta_stride[i] = c.meta_stride[i + HALF] = vq;
            }
        }
        return c;
    }
#pragma unroll
    for (int i = 0; i < S::NMETA; ++i) {
        // Lanes past the end reload the last float4 (never stored), so every
        // load is unconditional.
        const int e = min(lane + 64 * i, 2 * kq + 2 * vq - 1);
        if (e < kq) {
            c.meta[i] = reinterpret_cast<const float4*>(a.k_scale + cid0 * S::D) + e;
            c.meta_stride[i] = kq;
        } else if (e < 2 * kq) {
            c.meta[i] = reinterpret_cast<const float4*>(a.k_zero + cid0 * S::D) + (e - kq);
            c.meta_stride[i] = kq;
        } else if (e < 2 * kq + vq) {
            c.meta[i] = reinterpret_cast<const float4*>(a.v_scale + cid0 * NG * S::G) + (e - 2 * kq);
            c.meta_stride[i] = vq;
        } else {
            c.meta[i] = reinterpret_cast<const float4*>(a.v_zero + cid0 * NG * S::G) +
                        (e - 2 * kq - vq);
            c.meta_stride[i] = vq;
        }
    }
    return c;
}

// Issues the loads of chunk c (relative to the wave's (b, kv-head)).
// Streaming (nontemporal) loads: every code word, scale and zero is read once
// per launch, so keeping them out of L2 and the MALL costs nothing; measured
// 1-2 % faster at 8K context (B=64, 32/8 heads), 2-3 % at 128K (split-K) and
// 12 % at 4K with B=16 and 32 heads, where the 336 MB store would otherwise
// half fit the MALL and evict itself.
// The key codes and metadata (load_chunk_km) and the value codes
// (load_chunk_v) are issued separately: a ring slot's key codes and metadata
// are consumed one step before its value codes.
template <class S>
__device__ __forceinline__ void load_chunk_km(ChunkRegs<S>& r, const ChunkSrc<S>& src, int c) {
    const uint32_t* kc = src.kc + (int64_t)c * (64 * S::NP);
#pragma unroll
    for (int i = 0; i < S::NP; ++i) r.kc[i] = __builtin_nontemporal_load(kc + i);
#pragma unroll
    for (int i = 0; i < S::NMETA; ++i) {
        const kivi_f4v x = __builtin_nontemporal_load(
            reinterpret_cast<const kivi_f4v*>(src.meta[i] + (int64_t)c * src.meta_stride[i]));
        r.meta[i] = make_float4(x.x, x.y, x.z, x.w);
    }
}
template <class S>
__device__ __forceinline__ void load_chunk_v(ChunkRegs<S>& r, const ChunkSrc<S>& src, int c) {
    const uint32_t* vc = src.vc + (int64_t)c * (64 * S::NP);
#pragma unroll
    for (int i = 0; i < S::NP; ++i) r.vc[i] = __builtin_nontemporal_load(vc + i);
}
template <class S>
__device__ __forceinline__ void load_chunk(ChunkRegs<S>& r, const ChunkSrc<S>& src, int c) {
    const uint32_t* kc = src.kc + (int64_t)c * (64 * S::NP);
    const uint32_t* vc = src.vc + (int64_t)c * (64 * S::NP);
#pragma unroll
    for (int i = 0; i < S::NP; ++i) {
        r.kc[i] = __builtin_nontemporal_load(kc + i);
        r.vc[i] = __builtin_nontemporal_load(vc + i);
    }
#pragma unroll
    for (int i = 0; i < S::NMETA; ++i) {
        const kivi_f4v x = __builtin_nontemporal_load(
            reinterpret_cast<const kivi_f4v*>(src.meta[i] + (int64_t)c * src.meta_stride[i]));
        r.meta[i] = make_float4(x.x, x.y, x.z, x.w);
    }
}

// LDS float4 slots where a paired lane stages its i-th scale and zero float4
// ([ks | kz | vs | vz] order, meta_slot spacing), or -1 past the end.
// Fixed per wave: computed once.
template <class S>
struct PairSlots {
    int sc[S::NMETA / 2 > 0 ? S::NMETA / 2 : 1], zr[S::NMETA / 2 > 0 ? S::NMETA / 2 : 1];
};
template <class S>
__device__ __forceinline__ PairSlots<S> pair_slots(int lane, int NG) {
    PairSlots<S> p;
    const int kq = S::D / 4, vq = NG * S::G / 4;
#pragma unroll
    for (int i = 0; i < S::NMETA / 2; ++i) {
        const int e = lane + 64 * i;
        const bool key = e < kq;
        p.sc[i] = e < kq + vq ? S::meta_slot(key ? e : kq + e) : -1;
        p.zr[i] = e < kq + vq ? S::meta_slot(key ? kq + e : kq + vq + e) : -1;
    }
    return p;
}

// Code-scale multipliers of the lane's i-th metadata float4 (its elements
// 0-1 and 2-3): a scale float4 covers the four consecutive channels or tokens
// 4e..4e+3, at operand positions k = 2(e%2) + i/2, and is multiplied by
// 2^(kCodeExp - kProdExp - 2k); zeros by 1.  e = lane + 64i, so e%2 is the
// lane's parity (the ks and vs arrays start at even float4s).
template <class S, bool PAIRED>
__device__ __forceinline__ float2 meta_mul(int lane, int i, int NG) {
    const float2 m = (lane & 1) ? make_float2(0x1p65f, 0x1p63f) : make_float2(0x1p69f, 0x1p67f);
    if constexpr (PAIRED) return m;
    const int kq = S::D / 4, vq = NG * S::G / 4;
    const int e = min(lane + 64 * i, 2 * kq + 2 * vq - 1);    // as chunk_src clamps it
    const bool scale = e < kq || (e >= 2 * kq && e < 2 * kq + vq);
    return scale ? m : make_float2(1.f, 1.f);
}

// Stages a chunk's metadata in LDS as [ks | kz | vs | vz] float4 slots
// (meta_slot), the scales multiplied by their code-scale factors (mul[i],
// from meta_mul).
template <class S, bool PAIRED>
__device__ __forceinline__ void stage_meta(const ChunkRegs<S>& r, float* MT, int lane, int NG,
                                           int meta_floats, const PairSlots<S>& ps,
                                           const float2* mul) {
    float4* mt = reinterpret_cast<float4*>(MT);
    auto scaled = [&](float4 x, float2 m) {
        return make_float4(x.x * m.x, x.y * m.x, x.z * m.y, x.w * m.y);
    };
    if constexpr (PAIRED) {
        constexpr int HALF = S::NMETA / 2;
#pragma unroll
        for (int i = 0; i < HALF; ++i) {
            const float4 sc = scaled(r.meta[i], mul[i]);
            if (ps.sc[i] >= 0) {
                mt[ps.sc[i]] = sc;
                mt[ps.zr[i]] = r.meta[i + HALF];
            }
        }
        return;
    }
    // Every lane stores: a lane past the end holds the last float4 (its load
    // was clamped to it, chunk_src) and writes those same bits to the last
    // slot.  A conditional store was the value's only use, so the compiler
    // moved the chunk's metadata load into the branch, right before the
    // store and behind a wait for every outstanding load (the prefetch
    // ring's included).
    const int n4 = meta_floats / 4;
#pragma unroll
    for (int i = 0; i < S::NMETA; ++i) {
        const int e = min(lane + 64 * i, n4 - 1);
        mt[S::meta_slot(e)] = scaled(r.meta[i], mul[i]);
    }
}

// NGC > 0: the number of value groups per token (D / Gv) is NGC at compile
// time, so the value operand of every n-block is known statically and its
// LDS reads can be issued ahead; NGC == 0 reads it from the launch.
// R16: the residual ring holds bf16 or fp16 (a.res_dt) instead of fp32.
template <class S, int NGC, bool R16, bool MASK>
__device__ void wave_path(unsigned char* smem, const AttnLaunch& a, int split, int kvh, int b) {
    constexpr int HG = S::HG, D = S::D, G = S::G, NSUB = S::NSUB, NB = G / 16;
    // Value operand items: (head, value group, TPI tokens).  8 tokens per
    // item where the chunk has at least 64 of them; otherwise 2, so that the
    // operand build spreads over the wave instead of leaving most lanes idle
    // (one value group per token at 4 query heads per kv head has 16 items
    // of 8 tokens; MHA with 4 groups has 16).  With 2 tokens an item's
    // (head, group) spans whole 16-lane rows (G/2 items, consecutive), whose
    // value corrections are summed across the row before they are staged.
    constexpr int NGI = NGC > 0 ? NGC : S::NGMAX;
    constexpr int TPI = HG * NGI * (G / 8) >= 64 ? 8 : 2;
    constexpr int NSEG = G / TPI;                       // items per (head, group)
    constexpr int NSEGV = TPI == 8 ? NSEG : NSEG / 16;   // staged corrections per (head, group)
    constexpr int NEV = (HG * NSEG * NGI + 63) / 64;    // items per lane
    static_assert(TPI == 8 || NSEG % 16 == 0, "two-token items fill whole 16-lane rows");
    // wave-uniform in an SGPR: chunk ranges, ring indices and branches on
    // them stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int lane = threadIdx.x % kWave;
    const int NG = NGC > 0 ? NGC : D / a.Gv;
    const int Gv = NGC > 0 ? D / NGC : a.Gv;
    constexpr bool PAIRED = paired_meta<S>(NGC);
    const int64_t bh = (int64_t)b * a.Hkv + kvh;
    // Left padding: context positions before kv_lo take no weight (0: none).
    const int kv_lo = __builtin_amdgcn_readfirstlane(a.kv_start ? a.kv_start[b] : 0);
    // Any other padding pattern (MASK instances only): this sequence's
    // hidden-position bits (AttnLaunch::hidden), one word per 32 positions.
    const uint32_t* hid_row = MASK ? a.hidden + b * a.hidden_stride : nullptr;
    static_assert(G % 32 == 0, "chunks and residual passes hold whole hidden-position words");

    unsigned char* wl = smem + wave * S::wave_lds(NG);
    uint16_t* WA = reinterpret_cast<uint16_t*>(wl + S::OFF_WA);
    uint16_t* PA = reinterpret_cast<uint16_t*>(wl + S::OFF_PA);
    float* PL = reinterpret_cast<float*>(wl + S::off_pl(NG));      // [2][HG][G]
    float* AL = reinterpret_cast<float*>(wl + S::off_al(NG));      // [2][16]
    float* VB = reinterpret_cast<float*>(wl + S::off_vb(NG));
    float* MT = reinterpret_cast<float*>(wl + S::off_mt(NG));      // [2][meta]
    const int meta_floats = S::meta_floats(NG);
    const int meta_stride = S::meta_stride(NG);

    // Residual pass buffers (scaled q of the group, per-wave probabilities)
    // after the merge slots, and the combined residual state at the end.
    float* qres = reinterpret_cast<float*>(smem + S::qres_off(NG));             // [HG][D]
    float* rstate = reinterpret_cast<float*>(smem + S::res_off(NG));
    // ---- launch prologue -----------------------------------------------------
    // Every load the prologue needs is issued up front, in the order of use:
    // the new token (if any), the query, this lane's query channels for the
    // key operand builds, then the first PF chunks of the wave's prefetch
    // ring.  The barrier fences LDS only, so the ring's loads stay in flight
    // across it: the prologue costs one memory round trip, shared with the
    // first chunks.
    //
    // The new token is read from its own tensor by the residual pass below;
    // the first split also files it in the ring for later launches (nothing
    // in this launch reads that ring slot).  Lane e < D/4 of the first
    // split's last wave moves four elements of each row.  A wave waits for
    // its stores to complete before it reuses their data registers (one
    // memory round trip); the last wave holds the fewest chunks, so the wait
    // mostly stays off the critical path.
    const bool has_new = a.k_new != nullptr;
    const int64_t new_row = (int64_t)b * a.new_sb + (int64_t)kvh * a.new_sh;   // element offset
    using Quad = typename std::conditional<R16, uint2, uint4>::type;
    const bool copy_new = has_new && split == 0 && wave == kWaves - 1 && lane < D / 4;
    Quad kn{}, vn{};
    if (copy_new) {
        kn = static_cast<const Quad*>(a.k_new)[new_row / 4 + lane];
        vn = static_cast<const Quad*>(a.v_new)[new_row / 4 + lane];
    }
    // Query rows (QueryRows): padding rows read the last real row and are
    // zeroed after the load, so no load sits in a branch.
    constexpr int QN = (HG * D + kBlock - 1) / kBlock;
    const int n_real = a.qr.qlen * a.qr.hg;
    float qt[QN];
#pragma unroll
    for (int i = 0; i < QN; ++i) {
        const int e = min((int)threadIdx.x + i * kBlock, HG * D - 1);
        const int v = e / D;
        const float x = a.q[a.qr.row(b, kvh, min(v, n_real - 1), a.Hq, D) + e % D];
        qt[i] = v < n_real ? x : 0.f;
    }
    // W-prep lane: head wh, channels [wseg*CPL, +CPL).
    const bool wlane = lane < HG * S::LPH;
    const int wh = lane / S::LPH, wseg = lane % S::LPH;
    const float* qw = a.q + a.qr.row(b, kvh, min(wh, n_real - 1), a.Hq, D) + wseg * S::CPL;
    float qv[S::CPL];
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) qv[i] = wlane ? qw[i] : 0.f;
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) qv[i] = wh < n_real ? qv[i] : 0.f;
    // Keeps the query loads ahead of the ring's: the query's LDS stores then
    // wait for the query alone.
    asm volatile("" ::: "memory");

    // Residual passes are dealt whole, in reverse wave order (chunks are
    // dealt from wave 0, so the waves that may hold one chunk fewer take the
    // extra passes).  With res_waves == 1 the last wave of each workgroup
    // takes all of its split's passes while the other three stream chunks.
    const bool res_one = a.res_waves == 1;
    const int n_res_waves = a.n_qsplits * (res_one ? 1 : kWaves);
    const int widx = res_one ? (wave == kWaves - 1 ? n_res_waves - 1 - split : n_res_waves)
                             : n_res_waves - 1 - (split * kWaves + wave);
    const int n_pass = (a.res_len + kResPass - 1) / kResPass;
    const int pbase = n_pass / n_res_waves, pextra = n_pass % n_res_waves;
    // passes of this split's last wave when it alone takes them
    const int split_passes = pbase + (n_res_waves - 1 - split < pextra ? 1 : 0);

    // The workgroup's chunks [g_begin, g_end) are dealt to its waves in turn
    // (wave w takes g_begin + w + kWaves*j): the four waves then read
    // neighbouring chunks, which streams from HBM measurably faster than four
    // separate contiguous ranges.  When the last wave takes the whole
    // residual window (res_waves == 1), the first 3*early chunks are dealt to
    // the other three waves only, while it works on the window.  The dealing
    // is fixed per launch shape, so results are bit-for-bit reproducible.
    const int g_begin = split * kWaves * a.chunks_per_wave;
    const int g_end = min(g_begin + kWaves * a.chunks_per_wave, a.n_chunks);
    const int g_cnt = max(0, g_end - g_begin);
    // (0 when the context has no chunk yet: the ring's loads then read chunk 0
    // of the store, in bounds, and no step uses them)
    const int c_last = max(g_end - 1, 0);
    // early chunks per other wave: early_per_pass_x2 / 2 per pass, rounded
    const int early = min((a.early_per_pass_x2 * split_passes + 1) / 2, a.chunks_per_wave / 2);
    const int s_early = res_one ? min((kWaves - 1) * early, g_cnt) : 0;
    const int n_early = wave < kWaves - 1 ? (s_early - wave + kWaves - 2) / (kWaves - 1) : 0;
    const int n_mine = n_early + max(0, (g_cnt - s_early - wave + kWaves - 1) / kWaves);
    const int early_base = g_begin + wave;                               // + 3j
    const int late_base = g_begin + s_early + wave - kWaves * n_early;   // + 4j
    // the wave's j-th chunk, or -1 past its last
    auto chunk_of = [&](int j) {
        return j >= n_mine ? -1
                           : j < n_early ? early_base + (kWaves - 1) * j : late_base + kWaves * j;
    };
    constexpr int PF = S::PF;
    ChunkRegs<S> buf[PF];
    int cid[PF];     // the chunk in each ring slot; -1 past the end (its load re-reads c_last)
    const ChunkSrc<S> src = chunk_src<S, PAIRED>(a, bh * a.Cmax, lane, NG);
    const PairSlots<S> pslots = pair_slots<S>(lane, NG);
    float2 smul[S::NMETA];
#pragma unroll
    for (int i = 0; i < S::NMETA; ++i) smul[i] = meta_mul<S, PAIRED>(lane, i, NG);
    // Hidden-position words of the wave's chunks (launches with hidden
    // positions only): lane l holds those of the wave's chunk l, so a step
    // reads its words with readlane.  A scalar load per step made each step
    // wait for it at its next LDS wait (config 4: 103 -> 118 us); it remains
    // only for a wave's chunks past its 64th.
    uint32_t hid_lane[G / 32];
    if constexpr (MASK) {
        const int c = chunk_of(lane);
#pragma unroll
        for (int i = 0; i < G / 32; ++i)
            hid_lane[i] = c >= 0 ? hid_row[(int64_t)c * (G / 32) + i] : 0u;
    }
    int hid_j = 0;       // the wave's chunk index of the next kside call
    // (the launch gives every workgroup at least one chunk, or the store room
    // for chunk 0, so c_last is a readable chunk and these loads need no
    // branch: a branch here would make the compiler wait for them before the
    // query's LDS stores)
#pragma unroll
    for (int k = 0; k < PF; ++k) {
        cid[k] = chunk_of(k);
        load_chunk<S>(buf[k], src, cid[k] >= 0 ? cid[k] : c_last);
    }
    int next_j = PF;     // the wave's next chunk to load
#pragma unroll
    for (int i = 0; i < QN; ++i) {
        const int e = threadIdx.x + i * kBlock;
        if (e < HG * D) qres[e] = qt[i] * a.qscale;
    }
    lds_barrier();
    // After the barrier, so that no wave waits for these stores before it.
    if (copy_new) {
        const int64_t o = ((int64_t)bh * a.Rcap + a.new_slot) * (D / 4) + lane;
        static_cast<Quad*>(const_cast<void*>(a.k_res))[o] = kn;
        static_cast<Quad*>(const_cast<void*>(a.v_res))[o] = vn;
    }
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) qv[i] *= a.qscale;

    f32x4_t O[S::NBV];
#pragma unroll
    for (int i = 0; i < S::NBV; ++i) O[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const int gq = lane / 16, col = lane % 16;
    // Value A operands: row 2h / 2h+1 = hi / lo of head h; this lane reads
    // row col (or the zero row).
    const int arow = col < 2 * HG ? col : 2 * HG;
    // Key A operands: with three pieces, row 4h + p holds piece p of head h
    // and row 4h + 3 reads the zero row, so a lane's four output rows
    // (4gq..4gq+3) are the pieces of one head, gq; with two, row 2h + p, and
    // a lane's output rows hold heads 2gq and 2gq+1.  Stored compactly as
    // rows KP*h + p, the zero row last.
    constexpr int KP = S::KP, HPL = KP == 3 ? 1 : 2;   // key-side heads per lane
    const int karow = KP == 3 ? ((col % 4 < 3 && col / 4 < HG) ? 3 * (col / 4) + col % 4
                                                               : S::KROWS)
                              : arow;
    auto khead = [&](int e) { return KP == 3 ? gq : 2 * gq + e; };
    // the lane's LDS addresses in the chunk loop: key operand rows written
    // (W-prep lanes) and read, the value operand rows read, the probability
    // rows written
    uint16_t* const wa_w = pin_lds<S::PIN>(WA + (KP * wh) * S::WA_ROW + wseg * S::CPL);
    const uint16_t* const wa_r = pin_lds<S::PIN>(WA + karow * S::WA_ROW + 8 * gq);
    const uint16_t* const pa_r = pin_lds<S::PIN>(PA + arow * S::PA_ROW + 8 * gq);
    float* const pl_w = pin_lds<S::PIN>(PL + khead(0) * S::PL_ROW + col);
    // online-softmax state of the lane's key-side heads
    float m_run[HPL], l_part[HPL], m_thr[HPL];     // m_thr = m_run + kRescaleThreshold
    bool hvalid[HPL];
#pragma unroll
    for (int e = 0; e < HPL; ++e) {
        m_run[e] = -INFINITY;
        m_thr[e] = -INFINITY;
        l_part[e] = 0.f;
        hvalid[e] = khead(e) < HG;
    }
    float vb[NEV];
#pragma unroll
    for (int it = 0; it < NEV; ++it) vb[it] = 0.f;
    const int n_items = HG * NSEG * NG;

    const SplitConsts spc = split_consts();

    // ---- phases of one chunk --------------------------------------------------
    // Key A operand: rows KP*h + p = piece p of q[h,d]*ks'[d] (ks' the staged,
    // code-scaled key scale).  Returns the lane's part of the key correction,
    // sum_d q[h,d]*kz[d] over its channels (0 on lanes that build nothing).
    // Float offsets (within one metadata buffer) of this lane's ks / kz float4s.
    int wks[S::CPL / 4 > 0 ? S::CPL / 4 : 1], wkz[S::CPL / 4 > 0 ? S::CPL / 4 : 1];
#pragma unroll
    for (int i = 0; i < (S::CPL >= 4 ? S::CPL / 4 : 1); ++i) {
        const int s0 = (wseg * S::CPL) / 4 + i;
        wks[i] = 4 * S::meta_slot(s0) + (S::CPL >= 4 ? 0 : (wseg * S::CPL) % 4);
        wkz[i] = 4 * S::meta_slot(D / 4 + s0) + (S::CPL >= 4 ? 0 : (wseg * S::CPL) % 4);
    }
    auto wprep = [&](auto slot_c) -> float {
        constexpr int slot = decltype(slot_c)::value;
        if (!wlane) return 0.f;
        const float* mt = MT + slot * meta_stride;
        float ks[S::CPL], kz[S::CPL];
        if constexpr (S::CPL % 4 == 0) {
#pragma unroll
            for (int i = 0; i < S::CPL / 4; ++i) {
                const float4 a4 = *reinterpret_cast<const float4*>(mt + wks[i]);
                const float4 z4 = *reinterpret_cast<const float4*>(mt + wkz[i]);
                ks[4 * i] = a4.x; ks[4 * i + 1] = a4.y; ks[4 * i + 2] = a4.z; ks[4 * i + 3] = a4.w;
                kz[4 * i] = z4.x; kz[4 * i + 1] = z4.y; kz[4 * i + 2] = z4.z; kz[4 * i + 3] = z4.w;
            }
        } else {
            const float2 a2 = *reinterpret_cast<const float2*>(mt + wks[0]);
            const float2 z2 = *reinterpret_cast<const float2*>(mt + wkz[0]);
            ks[0] = a2.x; ks[1] = a2.y;
            kz[0] = z2.x; kz[1] = z2.y;
        }
        // pieces [KP][CPL/2] of the lane's channel pairs (hi, mid, lo or hi, lo)
        uint32_t pc[KP][S::CPL / 2];
        float corr = 0.f;
#pragma unroll
        for (int j = 0; j < S::CPL / 2; ++j) {
            const float xa = qv[2 * j] * ks[2 * j], xb = qv[2 * j + 1] * ks[2 * j + 1];
            if constexpr (KP == 3) split3_pair(xa, xb, pc[0][j], pc[1][j], pc[2][j], spc);
            else split_pair(xa, xb, pc[0][j], pc[1][j], spc);
            corr = fmaf(qv[2 * j], kz[2 * j], corr);
            corr = fmaf(qv[2 * j + 1], kz[2 * j + 1], corr);
        }
        // head wh's rows KP*wh + p, this lane's channels
#pragma unroll
        for (int pi = 0; pi < KP; ++pi) {
            uint16_t* rp = wa_w + pi * S::WA_ROW;
            if constexpr (S::CPL % 8 == 0) {
#pragma unroll
                for (int j = 0; j < S::CPL / 8; ++j)
                    *reinterpret_cast<u32x4_t*>(rp + 8 * j) =
                        u32x4_t{pc[pi][4 * j], pc[pi][4 * j + 1], pc[pi][4 * j + 2], pc[pi][4 * j + 3]};
            } else {
#pragma unroll
                for (int j = 0; j < S::CPL / 2; ++j) reinterpret_cast<uint32_t*>(rp)[j] = pc[pi][j];
            }
        }
        return corr;
    };
    // The key correction of each of the lane's key-side heads (khead(e)),
    // summed over that head's W-prep lanes (wh*LPH .. wh*LPH+LPH-1).  With 16
    // per head they are the DPP row of the head, which (three key pieces:
    // lane group gq = head gq) is where its scores are; with 8 (8 query
    // heads per kv head) half rows, heads 2gq and 2gq+1 being the two halves
    // of row gq; with 32 or 64, whole rows combined through readlane.  Every
    // lane takes part (wave-uniform control flow).
    auto head_corr = [&](float part, float* kc) {
        if constexpr (S::LPH == 16) {
            kc[0] = row_sum16(part);
        } else if constexpr (S::LPH == 8) {
            float v = part + dpp<0xB1>(part);          // quad_perm [1,0,3,2]
            v += dpp<0x4E>(v);                           // quad_perm [2,3,0,1]
            v += dpp<0x141>(v);                          // row_half_mirror: the half row
            const float other = dpp<0x128>(v);           // row_ror 8: the other half
            kc[0] = col < 8 ? v : other;
            kc[1] = col < 8 ? other : v;
        } else {
            const float r = row_sum16(part);
            const float c01 = lane_f(r, 0) + lane_f(r, 16), c23 = lane_f(r, 32) + lane_f(r, 48);
            kc[0] = HG == 1 ? c01 + c23 : (gq == 0 ? c01 : c23);
        }
    };
    static_assert(S::LPH == 16 || S::LPH == 8 || HG <= 2, "key correction lanes");
    static_assert(S::LPH != 16 || KP == 3, "16 correction lanes per head need one head per lane");

    // Scores of the chunk's G tokens (matrix cores), then the online softmax:
    // lane group gq holds heads 2gq, 2gq+1.  Returns whether any running max
    // moved (then O and l are already rescaled and AL[slot] holds the factors).
    // `chunk` is the chunk's index: its tokens before kv_lo (a left-padded
    // sequence) and those its hidden-position bits name get score -inf and
    // weight 0, on a wave-uniform branch that unpadded sequences never take.
    // kc: the key corrections of the lane's key-side heads (head_corr).
    auto kside = [&](const ChunkRegs<S>& r, auto slot_c, int chunk, const float* kc) -> bool {
        constexpr int slot = decltype(slot_c)::value;
        bf16x8_t Aw[S::KS];
#pragma unroll
        for (int ks = 0; ks < S::KS; ++ks)
            Aw[ks] = *reinterpret_cast<const bf16x8_t*>(wa_r + 32 * ks);
        f32x4_t Sc[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < S::KS; ++ks) {
                const uint32_t word = r.kc[ks * NSUB + nb / 2];
                acc = mfma(Aw[ks], (nb % 2) == 0 ? unpack_codes<0>(word) : unpack_codes<1>(word),
                           acc);
            }
            Sc[nb] = acc;
        }
        // A head's running max moves only when its chunk max exceeds it by
        // more than the threshold; that happens iff some lane holds a score
        // above m_run + threshold, so the 16-lane row max is taken only then.
        float sc[HPL][NB], alpha[HPL];
        bool over = false;
#pragma unroll
        for (int e = 0; e < HPL; ++e) {
            alpha[e] = 1.f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                sc[e][nb] = fmaf(KP == 3 ? (Sc[nb][2] + Sc[nb][1]) + Sc[nb][0]
                                         : Sc[nb][2 * e] + Sc[nb][2 * e + 1],
                                 kProdScale, kc[e]);
        }
        const int n_masked = kv_lo - chunk * G;       // leading tokens hidden by padding
        // MASK: the chunk's hidden-position words (wave-uniform; kside runs
        // once per chunk of the wave, in order)
        uint32_t hid[G / 32];
        bool masked = n_masked > 0;                           // wave-uniform
        if constexpr (MASK) {
            uint32_t hid_any = 0;
#pragma unroll
            for (int i = 0; i < G / 32; ++i) {
                hid[i] = hid_j < 64 ? __builtin_amdgcn_readlane(hid_lane[i], hid_j)
                                    : hid_row[chunk * (G / 32) + i];
                hid_any |= hid[i];
            }
            ++hid_j;
            masked = masked || hid_any != 0;
        }
        // token 16*nb + col of the chunk takes no weight
        auto tok_hidden = [&](int nb) {
            if constexpr (MASK)
                return 16 * nb + col < n_masked || ((hid[nb / 2] >> (16 * (nb % 2) + col)) & 1u);
            else
                return 16 * nb + col < n_masked;
        };
        if (__builtin_expect(masked, 0)) {
#pragma unroll
            for (int e = 0; e < HPL; ++e) {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) sc[e][nb] = tok_hidden(nb) ? -INFINITY : sc[e][nb];
            }
        }
#pragma unroll
        for (int e = 0; e < HPL; ++e) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) over |= hvalid[e] && sc[e][nb] > m_thr[e];
        }
        const bool any = __builtin_amdgcn_ballot_w64(over) != 0;
        if (__builtin_expect(any, 0)) {
#pragma unroll
            for (int e = 0; e < HPL; ++e) {
                float cm = sc[e][0];
#pragma unroll
                for (int nb = 1; nb < NB; ++nb) cm = fmaxf(cm, sc[e][nb]);
                cm = row_max16(cm);
                if (hvalid[e] && cm > m_thr[e]) {
                    alpha[e] = exp2_fast(m_run[e] - cm);
                    m_run[e] = cm;
                    m_thr[e] = cm + kRescaleThreshold;
                }
            }
#pragma unroll
            for (int e = 0; e < HPL; ++e) {
                l_part[e] *= alpha[e];
                if (col == 0 && hvalid[e]) AL[slot * 16 + khead(e)] = alpha[e];
            }
            // O's rows (value side) are heads 2gq, 2gq+1 of the lane; with one
            // key-side head per lane their factors come through AL.
            if constexpr (KP == 3) {
                wave_sync();
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int h = 2 * gq + e;
                    const float f = h < HG ? AL[slot * 16 + h] : 1.f;
#pragma unroll
                    for (int nb = 0; nb < S::NBV; ++nb) {
                        O[nb][2 * e] *= f;
                        O[nb][2 * e + 1] *= f;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
#pragma unroll
                    for (int nb = 0; nb < S::NBV; ++nb) {
                        O[nb][2 * e] *= alpha[e];
                        O[nb][2 * e + 1] *= alpha[e];
                    }
                }
            }
        }
        float* pl = pl_w + slot * (HG * S::PL_ROW);
        float pv[HPL][NB];
#pragma unroll
        for (int e = 0; e < HPL; ++e) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) pv[e][nb] = exp2_fast(sc[e][nb] - m_run[e]);
        }
        // (a hidden token's weight is 0 even while the running max is -inf)
        if (__builtin_expect(masked, 0)) {
#pragma unroll
            for (int e = 0; e < HPL; ++e) {
#pragma unroll
                for (int nb = 0; nb < NB; ++nb) pv[e][nb] = tok_hidden(nb) ? 0.f : pv[e][nb];
            }
        }
#pragma unroll
        for (int e = 0; e < HPL; ++e) {
            float lsum = 0.f;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                lsum += pv[e][nb];
                if (hvalid[e]) pl[(khead(e) - khead(0)) * S::PL_ROW + 16 * nb] = pv[e][nb];
            }
            l_part[e] += lsum;
        }
        return any;
    };

    // Value A operands: rows 2h / 2h+1 = hi / lo of p[h,t]*vs'[t,g] for each
    // group g (vs' the staged, code-scaled value scale), one item = (head,
    // group, TPI tokens); value corrections p*vz.  Item geometry is fixed per
    // lane: LDS offsets are computed once here.
    int it_valid[NEV], it_h[NEV], it_vb[NEV];
    const float* it_pl[NEV];      // the item's probabilities in PL slot 0
    uint16_t* it_pa[NEV];         // the item's hi row in the value A operand
    int it_mv[NEV], it_mv2[NEV], it_mz[NEV], it_mz2[NEV];
    // 8-token items are numbered so that the 16 lanes of each ds_read_b128
    // cycle take 16 consecutive items: lanes {0-3, 12-15, 20-27} -> 0-15 and
    // {4-11, 16-19, 28-31} -> 16-31 of each half-wave.  2-token items are
    // lane-ordered (their (head, group) rows must be DPP rows).
    const int ilane = TPI == 8 ? item_lane(lane) : lane;
#pragma unroll
    for (int it = 0; it < NEV; ++it) {
        const int e = ilane + 64 * it;
        const int h = e / (NSEG * NG), rem = e % (NSEG * NG);
        const int g = rem / NSEG, seg = rem % NSEG;
        it_valid[it] = e < n_items;
        it_h[it] = h;
        it_pl[it] = pin_lds<S::PIN>(PL + min(h, HG - 1) * S::PL_ROW + TPI * seg);
        // staged value correction: one per item, or per 16-item row
        it_vb[it] = TPI == 8 ? e : (seg % 16 == 0 ? (h * NG + g) * NSEGV + seg / 16 : -1);
        const int fv = 2 * D + g * G + TPI * seg;          // float index of vs
        if constexpr (TPI == 8) {
            it_mv[it] = 4 * S::meta_slot(fv / 4);          // vs[0..3]; +4 slot for [4..7]
            it_mv2[it] = 4 * S::meta_slot(fv / 4 + 1);
            it_mz[it] = 4 * S::meta_slot((fv + NG * G) / 4);    // vz
            it_mz2[it] = 4 * S::meta_slot((fv + NG * G) / 4 + 1);
        } else {                                           // a float2 within one slot
            it_mv[it] = 4 * S::meta_slot(fv / 4) + fv % 4;
            it_mz[it] = 4 * S::meta_slot((fv + NG * G) / 4) + (fv + NG * G) % 4;
            it_mv2[it] = it_mz2[it] = 0;
        }
        it_pa[it] = pin_lds<S::PIN>(PA + min(g, NG - 1) * S::PA_MAT + TPI * seg +
                                    2 * min(h, HG - 1) * S::PA_ROW);
    }
    auto pprep = [&](auto slot_c, bool any) {
        constexpr int slot = decltype(slot_c)::value;
        constexpr int pl_off = slot * (HG * S::PL_ROW);
        const float* mt = MT + slot * meta_stride;
#pragma unroll
        for (int it = 0; it < NEV; ++it) {
            if (TPI == 2 && it_valid[it]) {
                if (any) vb[it] *= AL[slot * 16 + it_h[it]];
                const float2 p = *reinterpret_cast<const float2*>(it_pl[it] + pl_off);
                const float2 vs = *reinterpret_cast<const float2*>(mt + it_mv[it]);
                const float2 vz = *reinterpret_cast<const float2*>(mt + it_mz[it]);
                uint32_t h2, l2;
                split_pair(p.x * vs.x, p.y * vs.y, h2, l2, spc);
                vb[it] = fmaf(p.y, vz.y, fmaf(p.x, vz.x, vb[it]));
                uint16_t* base = it_pa[it];
                *reinterpret_cast<uint32_t*>(base) = h2;
                *reinterpret_cast<uint32_t*>(base + S::PA_ROW) = l2;
            } else if (TPI == 8 && it_valid[it]) {
                if (any) vb[it] *= AL[slot * 16 + it_h[it]];
                const float4 pa = *reinterpret_cast<const float4*>(it_pl[it] + pl_off);
                const float4 pb = *reinterpret_cast<const float4*>(it_pl[it] + pl_off + 4);
                const float4 sa = *reinterpret_cast<const float4*>(mt + it_mv[it]);
                const float4 sb = *reinterpret_cast<const float4*>(mt + it_mv2[it]);
                const float4 za = *reinterpret_cast<const float4*>(mt + it_mz[it]);
                const float4 zb = *reinterpret_cast<const float4*>(mt + it_mz2[it]);
                const float p[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
                const float vs[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
                const float vz[8] = {za.x, za.y, za.z, za.w, zb.x, zb.y, zb.z, zb.w};
                u32x4_t hi, lo;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    uint32_t h2, l2;
                    split_pair(p[2 * j] * vs[2 * j], p[2 * j + 1] * vs[2 * j + 1], h2, l2, spc);
                    hi[j] = h2;
                    lo[j] = l2;
                }
                float acc = vb[it];
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    acc = fmaf(p[j], vz[j], acc);
                vb[it] = acc;
                uint16_t* base = it_pa[it];
                *reinterpret_cast<u32x4_t*>(base) = hi;
                *reinterpret_cast<u32x4_t*>(base + S::PA_ROW) = lo;
            }
        }
    };

    // o += P' . V-codes over the chunk's G tokens.
    auto vside = [&](const ChunkRegs<S>& r) {
#pragma unroll
        for (int kt = 0; kt < NSUB; ++kt) {
            int g_loaded = -1;
            bf16x8_t Ap;
#pragma unroll
            for (int nb = 0; nb < S::NBV; ++nb) {
                const int g = (16 * nb) / Gv;
                if (g != g_loaded) {
                    Ap = *reinterpret_cast<const bf16x8_t*>(pa_r + g * S::PA_MAT + 32 * kt);
                    g_loaded = g;
                }
                const uint32_t word = r.vc[kt * (D / 32) + nb / 2];
                O[nb] = mfma(Ap, (nb % 2) == 0 ? unpack_codes<0>(word) : unpack_codes<1>(word),
                             O[nb]);
            }
        }
    };

    bool any_cur = false;

    // ---- this wave's slice of the fp32 residual window ------------------------
    // Its own online-softmax state (mr, lr, orr), merged with the chunk state
    // in LDS.  Passes of 16 tokens; scores with 4 lanes per token (a quarter
    // of the channels each), the weighted sum with one float4 of channels per
    // lane and 64/(D/4) token slots; every load of a pass is issued up front.
    constexpr int F4 = D / 4;                 // float4 per token row
    constexpr int TS = 64 / F4;               // token slots in the value pass
    constexpr int KQ = D / 16;                // float4 per lane in the score pass
    {
        float mr[HG], lr[HG], orr[HG][4];
#pragma unroll
        for (int h = 0; h < HG; ++h) {
            mr[h] = -INFINITY;
            lr[h] = 0.f;
            orr[h][0] = orr[h][1] = orr[h][2] = orr[h][3] = 0.f;
        }
        float* pres = qres + HG * D + wave * HG * kResPass;                      // [HG][16]
        const int p0 = widx * pbase + min(widx, pextra);
        const int r0 = min(p0 * kResPass, a.res_len);
        const int r1 = min((p0 + pbase + (widx < pextra ? 1 : 0)) * kResPass, a.res_len);
        const int tk = lane / 4, qq = lane % 4;
        const int c4 = lane % F4, ts = lane / F4;
        const int r_lo = kv_lo - a.n_chunks * G;      // first visible window token
        // Four channels of a ring row widened to fp32.  The ring's width is
        // a template parameter (a run-time branch here would cost registers
        // at the kernel's peak, the prefetched chunks being live); bf16 vs
        // fp16 is a bit mask in the widening (load4_16).
        const uint32_t res_half = a.res_dt == kSrcF16 ? 0xffffffffu : 0u;
        auto load4 = [&](const void* p, int64_t i) {
            if constexpr (R16) return load4_16(p, i, res_half);
            else return load4_vec<kSrcF32>(p, i);
        };

        static_assert(kResPass == 16, "a pass's positions lie in one hidden-position word");
        for (int t0 = r0; t0 < r1; t0 += kResPass) {
            const int n = min(kResPass, r1 - t0);
            // MASK: the pass's hidden-position bits: positions n_chunks*G +
            // t0 .. + 15 lie in one word, from bit t0 % 32 (G is a multiple
            // of 32)
            uint32_t wh = 0u;
            if constexpr (MASK) wh = hid_row[(a.n_chunks * (G / 32)) + (t0 >> 5)] >> (t0 & 31);
            // scores: lane (tk, qq) takes channel quads qq, qq+4, ... of token tk's row
            const int ktok = t0 + min(tk, n - 1);          // index in the window
            int slot = a.res_start + ktok;
            slot = slot >= a.Rcap ? slot - a.Rcap : slot;
            const bool knew = has_new && ktok == a.res_len - 1;
            const int64_t krow = (knew ? new_row : ((int64_t)bh * a.Rcap + slot) * D) + 4 * qq;
            const void* kbase = knew ? a.k_new : a.k_res;
            float4 kv[KQ];
#pragma unroll
            for (int j = 0; j < KQ; ++j) kv[j] = load4(kbase, krow + 16 * j);
            // the pass's value rows are independent of the scores: load them
            // now so that a pass waits for HBM once
            float4 vv[kResPass / TS];
#pragma unroll
            for (int j = 0; j < kResPass / TS; ++j) {
                const int vtok = t0 + min(ts + TS * j, n - 1);
                int vs = a.res_start + vtok;
                vs = vs >= a.Rcap ? vs - a.Rcap : vs;
                const bool vnew = has_new && vtok == a.res_len - 1;
                vv[j] = load4(vnew ? a.v_new : a.v_res,
                              (vnew ? new_row : ((int64_t)bh * a.Rcap + vs) * D) + 4 * c4);
            }
            // MASK: token tk of the pass is real, not before kv_lo and not hidden
            bool tseen = false;
            if constexpr (MASK) tseen = tk < n && t0 + tk >= r_lo && !((wh >> tk) & 1u);
            float sres[HG];
#pragma unroll
            for (int h = 0; h < HG; ++h) {
                const float4* qh = reinterpret_cast<const float4*>(qres + h * D) + qq;
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < KQ; ++j) {
                    const float4 qv4 = qh[4 * j];
                    acc = fmaf(qv4.x, kv[j].x, acc);
                    acc = fmaf(qv4.y, kv[j].y, acc);
                    acc = fmaf(qv4.z, kv[j].z, acc);
                    acc = fmaf(qv4.w, kv[j].w, acc);
                }
                acc += dpp<0xB1>(acc);        // quad_perm [1,0,3,2]
                acc += dpp<0x4E>(acc);        // quad_perm [2,3,0,1]
                // row h sees the window's first qr.visible(h) tokens
                if constexpr (MASK)
                    sres[h] = tseen && t0 + tk < a.qr.visible(h, a.res_len) ? acc : -INFINITY;
                else
                    sres[h] = tk < n && t0 + tk >= r_lo && t0 + tk < a.qr.visible(h, a.res_len)
                                  ? acc : -INFINITY;
            }
#pragma unroll
            for (int h = 0; h < HG; ++h) {
                const float mnew = fmaxf(mr[h], wave_max(sres[h]));
                const float alpha = mr[h] == -INFINITY ? 0.f : exp2_fast(mr[h] - mnew);
                mr[h] = mnew;
                float p;
                if constexpr (MASK)
                    p = tseen && t0 + tk < a.qr.visible(h, a.res_len) ? exp2_fast(sres[h] - mnew)
                                                                       : 0.f;
                else
                    p = tk < n && t0 + tk >= r_lo && t0 + tk < a.qr.visible(h, a.res_len)
                            ? exp2_fast(sres[h] - mnew) : 0.f;
                lr[h] = lr[h] * alpha + 0.25f * wave_sum(p);    // each token sits in 4 lanes
                orr[h][0] *= alpha;
                orr[h][1] *= alpha;
                orr[h][2] *= alpha;
                orr[h][3] *= alpha;
                if (qq == 0) pres[h * kResPass + tk] = p;
            }
            wave_sync();
            // weighted sum of the values
#pragma unroll
            for (int j = 0; j < kResPass / TS; ++j) {
                const int tt = ts + TS * j;
#pragma unroll
                for (int h = 0; h < HG; ++h) {
                    const float p = tt < n ? pres[h * kResPass + tt] : 0.f;
                    orr[h][0] = fmaf(p, vv[j].x, orr[h][0]);
                    orr[h][1] = fmaf(p, vv[j].y, orr[h][1]);
                    orr[h][2] = fmaf(p, vv[j].z, orr[h][2]);
                    orr[h][3] = fmaf(p, vv[j].w, orr[h][3]);
                }
            }
            wave_sync();
        }
        // fold the token slots (lanes c4, c4 + F4, ... hold the same channels)
        // and park the slice's state in this wave's merge slot
#pragma unroll
        for (int sh = F4; sh < 64; sh <<= 1) {
#pragma unroll
            for (int h = 0; h < HG; ++h) {
#pragma unroll
                for (int i = 0; i < 4; ++i) orr[h][i] += __shfl_xor(orr[h][i], sh);
            }
        }
        // (res_waves == 1: the last wave's state is the workgroup's residual
        // state, written straight to rstate; nobody waits for it before the
        // final merge)
        float* rst = res_one ? rstate : merge_slot(smem, HG, D, wave);
        const bool keep = !res_one || wave == kWaves - 1;
        if (keep && lane < F4) {
#pragma unroll
            for (int h = 0; h < HG; ++h) {
#pragma unroll
                for (int i = 0; i < 4; ++i) rst[h * D + 4 * lane + i] = orr[h][i];
            }
        }
        if (keep && lane == 0) {
#pragma unroll
            for (int h = 0; h < HG; ++h) {
                rst[HG * D + h] = mr[h];
                rst[HG * D + HG + h] = lr[h];
            }
        }
    }
    if (!res_one) combine_residual<HG, D>(smem, rstate);

    // Zero the A operands once: the zero row and correction columns >= LPH
    // are never written and must read as 0.
    for (int e = lane; e < S::off_pl(NG) / 4; e += kWave) reinterpret_cast<uint32_t*>(wl)[e] = 0u;

    // ---- software-pipelined chunk loop ----------------------------------------
    // Step i finishes chunk i (value operands and o update) while it starts
    // chunk i+1 (metadata, key operands, scores, softmax): the two halves are
    // independent, so their latencies overlap, and each chunk costs two
    // wave-level LDS syncs.  Chunk data come from the ring of PF register
    // buffers, refilled PF chunks ahead (a slot past the end re-reads a valid
    // chunk, so no load is inside a branch and the compiler waits only for
    // the chunk about to be used).
    if (cid[0] >= 0) {
        stage_meta<S, PAIRED>(buf[0], MT, lane, NG, meta_floats, pslots, smul);
        wave_sync();
        float kc0[HPL];
        head_corr(wprep(Int<0>{}), kc0);
        wave_sync();
        any_cur = kside(buf[0], Int<0>{}, cid[0], kc0);
    }
    // Step i (of the wave's chunks, counted from 0) uses double-buffer
    // slot i & 1; PF is even, so within the unrolled ring the slot of step k
    // is k & 1, a compile-time constant.
    // `after_v` runs once the value products have read cur's value codes.
    auto step = [&](const ChunkRegs<S>& cur, const ChunkRegs<S>& nxt, bool has_next, auto slot_c,
                    int nxt_chunk, auto&& after_v) {
        constexpr int slot = decltype(slot_c)::value, nslot = slot ^ 1;
        if (has_next)
            stage_meta<S, PAIRED>(nxt, MT + nslot * meta_stride, lane, NG, meta_floats, pslots,
                                  smul);
        wave_sync();
        float kc[HPL];
        if (has_next) head_corr(wprep(Int<nslot>{}), kc);
        pprep(Int<slot>{}, any_cur);
        any_cur = false;            // vb now follows the current running max
        wave_sync();
        // A wave in its matrix-core phase (value MFMAs, then the next chunk's
        // scores and softmax) runs at a raised priority, so that when both
        // waves of a SIMD are ready the one whose MFMA chain and softmax gate
        // the next step goes first and the other's operand prep fills in.
        // Measured 3.3 % faster at config 4 and 5.5 % at config 5 (in-process
        // A/B); raising it around the ring loads, or over the prep phase
        // instead, did not help.
        __builtin_amdgcn_s_setprio(2);
        vside(cur);
        after_v();
        if (has_next) any_cur = kside(nxt, Int<nslot>{}, nxt_chunk, kc);
        __builtin_amdgcn_s_setprio(0);
    };
    static_assert(PF % 2 == 0, "the slot parity of a ring step must be static");

    // O accumulates sum_t (p vs) c (in units of 2^-64), which exceeds the
    // output by -sum_t p vz, the per-item correction kept in vb (with zeros
    // near a group's minimum, ~1.5 sum_t p vs).  Cancelled only at the end,
    // that excess lets O's rounding grow with the whole context: each chunk
    // adds ~2^-24 of it, which over long contexts of near-uniform weights
    // approaches the size of the output itself (measured 3e-3 relative at
    // 1025 chunks per wave when codes entered as 8 + c, a ~5x larger excess).
    // Folding vb into O every kFoldChunks chunks keeps the excess in O to
    // that of at most kFoldChunks chunks.  Called after a whole ring, where the
    // pending rescale (if the last scores moved the running max) is in AL
    // slot 0 and has not reached vb yet: it is applied here, and the next
    // pprep then scales zeros.
    constexpr int kFoldChunks = 16;
    constexpr int kFoldRings = kFoldChunks / PF > 0 ? kFoldChunks / PF : 1;
    // Stages the lanes' value corrections in VB ([h][g][NSEGV]) and clears
    // them; `rescale`: apply the pending rescale of AL slot 0 first.
    auto stage_vcorr = [&](bool rescale) {
#pragma unroll
        for (int it = 0; it < NEV; ++it) {
            float x = it_valid[it] ? (rescale && any_cur ? vb[it] * AL[it_h[it]] : vb[it]) : 0.f;
            if constexpr (TPI == 2) x = row_sum16(x);     // a row is one (head, group)
            if (it_valid[it] && it_vb[it] >= 0) VB[it_vb[it]] = x;
            vb[it] = 0.f;
        }
    };
    auto fold_vcorr = [&]() {
        wave_sync();
        stage_vcorr(true);
        wave_sync();
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int h = 2 * gq + e;
            if (h < HG) {
#pragma unroll
                for (int nb = 0; nb < S::NBV; ++nb) {
                    const float* pv = VB + (h * NG + (16 * nb + col) / Gv) * NSEGV;
                    float v = 0.f;
#pragma unroll
                    for (int sg = 0; sg < NSEGV; ++sg) v += pv[sg];
                    O[nb][2 * e] = fmaf(v, kProdUnit, O[nb][2 * e]);
                }
            }
        }
    };
    // The ring holds the wave's chunks in order, valid ones first.  The main
    // loop runs whole rings while every slot holds a chunk (no branch inside,
    // so the compiler schedules across the steps); the last partial ring is
    // the tail, which loads nothing.  Slot k is refilled with the chunk PF
    // ahead in two parts: its key codes and metadata, last used by the
    // previous step (stage_meta and kside of the slot's chunk), before step
    // k, and its value codes once step k's value products have read them.
    // The refill then leads its use by three steps for three quarters of
    // the bytes (two when the whole slot waited for the end of the step).
    int rings = 0;
    while (cid[PF - 1] >= 0) {
        static_for<0, PF>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            const int c_new = chunk_of(next_j++);
            const int c_ld = c_new >= 0 ? c_new : c_last;
            load_chunk_km<S>(buf[k], src, c_ld);
            step(buf[k], buf[(k + 1) % PF], k + 1 < PF || cid[0] >= 0, Int<k & 1>{},
                 cid[(k + 1) % PF], [&] { load_chunk_v<S>(buf[k], src, c_ld); });
            cid[k] = c_new;
        });
        if (++rings == kFoldRings) {
            rings = 0;
            fold_vcorr();
        }
    }
    static_for<0, PF - 1>([&](auto kc) {
        constexpr int k = decltype(kc)::value;
        if (cid[k] >= 0) step(buf[k], buf[k + 1], cid[k + 1] >= 0, Int<k & 1>{}, cid[k + 1], [] {});
    });
    // ---- wave state -> merge slot --------------------------------------------
    wave_sync();
    stage_vcorr(false);
    float l_tot[HPL];
#pragma unroll
    for (int e = 0; e < HPL; ++e) l_tot[e] = row_sum16(l_part[e]);
    wave_sync();
    // Gather this wave's value corrections before the merge slot (which
    // overlaps the per-wave LDS) is written.
    float vcorr[2][S::NBV];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int h = 2 * gq + e;
#pragma unroll
        for (int nb = 0; nb < S::NBV; ++nb) {
            float v = 0.f;
            if (h < HG) {
                const int g = (16 * nb + col) / Gv;
                const float* pv = VB + (h * NG + g) * NSEGV;
#pragma unroll
                for (int sg = 0; sg < NSEGV; ++sg) v += pv[sg];
            }
            vcorr[e][nb] = v;
        }
    }
    __syncthreads();
    float* slot = merge_slot(smem, HG, D, wave);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const int h = 2 * gq + e;
        if (h < HG) {
#pragma unroll
            for (int nb = 0; nb < S::NBV; ++nb)
                slot[h * D + 16 * nb + col] =
                    fmaf(O[nb][2 * e] + O[nb][2 * e + 1], kProdScale, vcorr[e][nb]);
        }
    }
#pragma unroll
    for (int e = 0; e < HPL; ++e) {
        if (col == 0 && hvalid[e]) {
            slot[HG * D + khead(e)] = m_run[e];
            slot[HG * D + HG + khead(e)] = l_tot[e];
        }
    }
    merge_and_store<HG, D, MASK>(smem, rstate, a, split, kvh, b);
}

// Occupancy target: three waves per SIMD for head_dim 64 with G=32 and up to
// 4 query heads per kv head (at four, with up to 2 query heads per kv head
// and 128 VGPRs, the key operands' third piece spilled: 16 % slower at B=16,
// 12/12 heads, 8K context; with 4, spills landed in the chunk loop: 85 us
// against 70 us at B=64, 32/8 heads); two where the 4-deep prefetch ring fits that
// register budget without spilling (head_dim 64, or head_dim 128 with up to
// 4 query heads per kv head), which measured faster than three waves with a
// 2-deep ring.  Head_dim 128 with 8 query heads per kv head and G=32 also
// runs two waves per SIMD, with a 2-deep ring (Shape::PF): two of its
// workgroups fit a CU's LDS.  With G=64 that workgroup needs more than half
// the LDS, so one workgroup runs per CU whatever its registers, and it keeps
// the full register file, as does head_dim 256 (one wave per SIMD).
template <int HG, int D, int G>
constexpr int attn_waves_per_eu() {
    return (D <= 64 && G <= 32 && HG <= 4) ? 3
           : (D <= 64 || (D <= 128 && (HG <= 4 || G <= 32))) ? 2 : 1;
}

template <int HG, int D, int G, int NGC, bool R16, bool MASK>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(attn_waves_per_eu<HG, D, G>())))
void attn_mfma_kernel(AttnLaunch a) {
    extern __shared__ __align__(16) unsigned char smem[];
    using S = Shape<HG, D, G>;
    // A workgroup puts one wave on each SIMD, so n waves per SIMD need n
    // workgroups' LDS on a CU (160 KB on gfx950).
    static_assert(attn_waves_per_eu<HG, D, G>() == 1 ||
                      attn_waves_per_eu<HG, D, G>() * S::lds(S::NGMAX) <= 160 * 1024,
                  "occupancy target exceeds the CU's LDS");
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
    wave_path<S, NGC, R16, MASK>(smem, a, split, kvh, b);
}

int max_lds_per_block() {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return 64 * 1024;
    return v;
}

template <int HG, int D, int G, int NGC, bool R16>
int launch_shape(const AttnLaunch& a, hipStream_t st) {
    using S = Shape<HG, D, G>;
    static const int lds_limit = max_lds_per_block();
    const int lds = S::lds(D / a.Gv);
    if (lds > lds_limit)
        return set_error(kErrUnsupported,
                         "decode attention with q_heads/kv_heads=%d, head_dim=%d, G=%d, "
                         "group_size_v=%d needs %d bytes of LDS per workgroup; the device "
                         "allows %d", HG, D, G, a.Gv, lds, lds_limit);
    const dim3 grid(a.n_splits, a.Hkv, a.B);
    // Launches with hidden positions run their own instances (MASK), so that
    // every other launch runs exactly the code it ran without mask support.
    // With the mask's code in the same instances, hipcc 7.2 scheduled a VALU
    // write into the dead zero-row element of an accumulating MFMA 8 wait
    // states after it, and the MFMA's later write of that register clobbered
    // the value: timing-dependent wrong scores at head_dim 64 with one query
    // head per kv head; keeping the element live moved the problem to run-to-
    // run differences at config 4.  The MASK instances were checked on their
    // own (every instance family, long contexts, repeated calls).
    if (a.hidden)
        attn_mfma_kernel<HG, D, G, NGC, R16, true><<<grid, kBlock, lds, st>>>(a);
    else
        attn_mfma_kernel<HG, D, G, NGC, R16, false><<<grid, kBlock, lds, st>>>(a);
    return check_launch("packed_decode_attention (mfma)");
}

// gfx950 LDS per workgroup.  Shapes whose fixed LDS need exceeds it are
// not instantiated (they could never launch).
constexpr int kMaxLdsBytes = 160 * 1024;

template <int HG, int D, int G, int NG>
constexpr bool lds_fits() {
    return Shape<HG, D, G>::lds(NG) <= kMaxLdsBytes;
}

// Value groups of 32 channels, one group per token, or (head_dim 128/256
// with 64- or 128-channel groups) the runtime count.
template <int HG, int D, int G, bool R16>
int launch_ng(const AttnLaunch& a, hipStream_t st) {
    if (a.Gv == 32) {
        if constexpr (lds_fits<HG, D, G, D / 32>())
            return launch_shape<HG, D, G, D / 32, R16>(a, st);
        return set_error(kErrUnsupported,
                         "decode attention with q_heads/kv_heads=%d, head_dim=%d, G=%d, "
                         "group_size_v=32 needs %d bytes of LDS per workgroup (at most %d)",
                         HG, D, G, Shape<HG, D, G>::lds(D / 32), kMaxLdsBytes);
    }
    if (a.Gv == D) return launch_shape<HG, D, G, 1, R16>(a, st);
    // (8 rows at head_dim 256, G = 64, would spill: the host plans at most 4
    // rows per launch there, so this instance is not built)
    if constexpr (D > 64 && !(HG == 8 && D == 256 && G == 64))
        return launch_shape<HG, D, G, 0, R16>(a, st);
    return set_error(kErrUnsupported, "group_size_v=%d with head_dim=%d", a.Gv, D);
}

template <int HG, int D, bool R16>
int launch_g(const AttnLaunch& a, hipStream_t st) {
    return a.G == 32 ? launch_ng<HG, D, 32, R16>(a, st) : launch_ng<HG, D, 64, R16>(a, st);
}

// Every kernel shape for one Hq/Hkv ratio and ring width.
template <int HG, bool R16>
int launch_d(const AttnLaunch& a, hipStream_t st) {
    switch (a.D) {
        case 64: return launch_g<HG, 64, R16>(a, st);
        case 128: return launch_g<HG, 128, R16>(a, st);
        default: return launch_g<HG, 256, R16>(a, st);
    }
}

}  // namespace
}  // namespace kivi
