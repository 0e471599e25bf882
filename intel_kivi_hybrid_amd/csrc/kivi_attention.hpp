// Internal interface between the decode-attention entry point
// (kivi_attention.hip) and its matrix-core kernel (kivi_attention_mfma.hpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kivi {

// Query rows of one launch.  A launch covers qlen query tokens and hg query
// heads of each kv head (heads h0 .. h0+hg-1 of the hg_all = Hq / Hkv that
// share it): the rows a workgroup computes for kv head kvh ("virtual heads"
// v) are query token i = v / hg and head kvh*hg_all + h0 + v % hg, so that
// v < qlen*hg are real rows and the rest padding (zero queries, never
// stored).  Both maps are tables of 4 bits per row (at most 8 rows), so any
// head ratio costs the kernels a shift and a mask.  Row v of batch b sits at
// q + b*q_bstride + (i*Hq + kvh*hg_all + h0 + h)*D, and its output likewise
// in out.  Query token i sees every quantised chunk and the first
// min(res_len, vis0 + i) tokens of the residual window (causal attention of
// the window's newest tokens; vis0 = res_len when every token sees all).
struct QueryRows {
    int qlen = 1, hg = 1;
    int hg_all = 1, h0 = 0;
    uint32_t row_tok = 0;     // bits 4v..4v+3: query token of row v
    uint32_t row_head = 0;    // bits 4v..4v+3: head of row v within the launch
    int64_t q_bstride = 0;
    int vis0 = 0;
    int rows = 1;            // HG: qlen*hg rounded up to a power of two (<= 8)
    __host__ __device__ int tok(int v) const { return (int)((row_tok >> (4 * v)) & 15u); }
    __host__ __device__ int64_t row(int b, int kvh, int v, int Hq, int D) const {
        const int h = (int)((row_head >> (4 * v)) & 15u);
        return (int64_t)b * q_bstride +
               ((int64_t)tok(v) * Hq + (int64_t)kvh * hg_all + h0 + h) * D;
    }
    __host__ __device__ bool real(int v) const { return v < qlen * hg; }
    __host__ __device__ int visible(int v, int res_len) const {
        const int n = vis0 + tok(v);
        return n < res_len ? n : res_len;
    }
};

struct AttnLaunch {
    const float* q;          // query rows (QueryRows)
    const uint8_t* k_codes;  // [B, Hkv, Cmax, G*D/4]
    const float* k_scale;    // [B, Hkv, Cmax, D]
    const float* k_zero;
    const uint8_t* v_codes;  // [B, Hkv, Cmax, G*D/4]
    const float* v_scale;    // [B, Hkv, Cmax, D/Gv, G]
    const float* v_zero;
    const void* k_res;       // [B, Hkv, Rcap, D] ring of element type res_dt
    const void* v_res;
    float* out;              // output rows (QueryRows)
    float* part_o;           // [B, Hkv, HG, n_splits, D] (n_splits > 1 only)
    float* part_ml;          // [B, Hkv, HG, n_splits, 2]
    int B, Hq, Hkv, D, G, Gv, Cmax, n_chunks, Rcap, res_start, res_len;
    int n_qsplits;           // workgroups per (b, kv-head)
    int chunks_per_wave;     // packed chunks per wave
    int res_waves;           // waves per workgroup that take residual passes (1: the last)
    int early_per_pass_x2;   // res_waves == 1: twice the chunks each other wave takes first per residual pass
    int n_splits;            // partial states per row (= n_qsplits)
    float qscale;            // softmax scale * log2(e)
    // Optional new token, the window's last (index res_len - 1): when k_new
    // is set the kernel reads that token from k_new / v_new (element
    // (b, h, d) at b*new_sb + h*new_sh + d, of the ring's type) and writes it
    // to ring slot new_slot, so no separate append launch is needed.
    const void* k_new = nullptr;
    const void* v_new = nullptr;
    int64_t new_sb = 0, new_sh = 0;
    int new_slot = 0;
    int res_dt = 0;          // ring element type: 0 fp32, 1 bf16, 2 fp16
    QueryRows qr;
    // Optional [B] first visible context position per sequence (a
    // left-padded batch): positions before kv_start[b] -- quantised or in
    // the window -- take no weight.  nullptr: every position is visible.
    const int32_t* kv_start = nullptr;
    // Optional per-sequence hidden positions (any padding pattern): bit p % 32
    // of word hidden[b * hidden_stride + p / 32] set hides context position p
    // of sequence b from every query token.  nullptr: none hidden.
    const uint32_t* hidden = nullptr;
    int64_t hidden_stride = 0;
};

// Bit p % 32 of a hidden-position row (see AttnLaunch::hidden).
__device__ __forceinline__ bool position_hidden(const uint32_t* row, int p) {
    return (row[p >> 5] >> (p & 31)) & 1u;
}

// Launches the matrix-core kernel (kLayoutMfma stores, Hq/Hkv in {1,2,4,8}).
// With n_splits == 1 it writes `out`; otherwise partials, which the caller
// merges.  The kernel templates live in kivi_attention_mfma.hpp; each
// Hq/Hkv ratio and ring width (fp32, or 16-bit: _r16) is instantiated in its
// own translation unit (kivi_attention_mfma_hg<N>[_r16].hip) so that the
// build compiles them in parallel.
int launch_attention_mfma(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg1(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg2(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg4(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg8(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg1_r16(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg2_r16(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg4_r16(const AttnLaunch& a, hipStream_t stream);
int launch_attention_mfma_hg8_r16(const AttnLaunch& a, hipStream_t stream);

// LDS bytes per workgroup of the matrix-core kernel for HG query heads per
// kv head, head_dim D, key group G and NG value groups per token (-1 for a
// shape it has no instance of).
int attention_mfma_lds_bytes(int HG, int D, int G, int NG);

}  // namespace kivi
