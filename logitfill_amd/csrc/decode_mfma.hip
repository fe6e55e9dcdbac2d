// Packed decode attention on the gfx950 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Reference semantics: src/logitfill/packed/reference.py:30-56 (dense dequantise,
// softmax attention over [history ; tail ; new]); replaces the CUDA kernel
// src/logitfill/packed/kernel.cu:112-190.  Shapes served: head_dim 128,
// page = Key group = 128 tokens, one Value group per token (v_group 128), int2
// Values, 1 <= g = n_q/n_kv <= 8.  Anything else runs the VALU kernel.
//
// Work: one workgroup (4 waves) per (split item, kv head).  Pages of the item
// are staged in LDS (double buffered through registers); each wave takes 32
// of a page's 128 tokens.
//
// Scores.  With the Key scale folded into the query once per page,
//     s[t][i] = sum_slot Qs[i][slot] * code[t][slot] + bias[i],
//     Qs = q * scaling * log2(e) * scale_slot,  bias = sum_c q_c * min_c,
// computed as S^T = Codes . Qs^T with the K dimension = the page's slots
// ordered tier by tier in blocks of 8 codes (an int2 word gives two blocks,
// an int4 word one, two int8 words one, eight fp16 values one); each K-step of
// 32 covers four blocks of one tier.  Codes become exact fp16 integers
// (magic-exponent OR, then -1024).  Qs is split hi + lo in fp16: columns
// 0..7 hold hi, columns 8..15 lo (the GQA group has at most 8 heads), and
// one DPP add recombines them, so the products carry ~22 bits.
//
// Values.  The S^T accumulator layout (lane: head n = lane%16, tokens
// 4*kb+r of the two 16-token tiles, kb = lane/16) is exactly the A-operand
// layout of O = P' . Codes_V with k = those 8 tokens, so probabilities feed
// the second MFMA without data movement.  P' = p * vscale is again split
// hi/lo across rows 0..7 / 8..15; the Value minimum enters through
// sum_t p_t * vmin_t.  Value codes are byte-transposed at staging (one dword
// = one byte column of 4 consecutive tokens) so each lane's 8 codes are two
// LDS dwords.
//
// Softmax: per wave online max/sum in the log2 domain; the 4 waves' partials
// merge in LDS; split items merge across workgroups (decode_common.hpp).
#include "decode_common.hpp"

namespace lf {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kMaxStage = 4;     // 16-byte staging chunks per thread per page

struct MfmaLayout {
    int kst[4];      // K-steps per tier
    int nblk[4];     // real 8-code blocks per tier
    int kfirst[4];   // first K-step of each tier
    int nb;          // padded blocks (4 per K-step)
    int nb_int;      // padded blocks of the integer tiers
    int w16p;        // fp16-tier row stride in LDS (multiple of 8)
    int off_qperm;   // [nb][8 heads][8] fp32: q * scaling*log2e for each slot (0 for padding)
    int off_qs;      // [nb][16][8] fp16: per-page Qs hi (rows 0..7) / lo (rows 8..15)
    int off_tt;      // tier table of this kv head: ranks -> channel ids (int16), per tier
    int off_small;   // bias partials [4][8], alpha [4][8], wave m/l/mv [4][3][8]
    int off_pbuf;    // residual probabilities [4][32][8] fp32
    int off_pb[2];   // page buffers
    int pb_kt[3];    // [128][words_t] u32 Key codes of tier t
    int pb_v16;      // [128][w16p] fp16 Key fp16 tier (zero padded)
    int pb_vt;       // [32 token groups][4][8] u32 byte-transposed Value codes
    int pb_vsc;      // [128] fp32 Value scale
    int pb_vmn;      // [128] fp32 Value min
    int pb_ksc;      // [nb_int][8] fp32 Key scale of each integer-tier slot (this page)
    int pb_kmn;      // [nb_int][8] fp32 Key min
    int seg_end[6];  // cumulative 16-byte chunks: K0, K1, K2, fp16 tier, v scale, v min
    int off_merge;    // merge scratch (aliases qperm/qs; free when the partial is stored)
    int merge_floats;
    int lds_bytes;
};

struct MfmaParams {
    DecodeParams p;
    MfmaLayout y;
};

__device__ __forceinline__ uint32_t lds_u32(const unsigned char* base, int byte) {
    return *reinterpret_cast<const uint32_t*>(base + byte);
}

// Slot (tier-local channel rank) of position ``pos`` (0..7) in local block ``lb``.
__device__ __forceinline__ int block_slot(int tier, int lb, int pos) {
    const int r = pos >> 1, odd = pos & 1;
    if (tier == 0) {  // int2: word lb/2, half lb%2; register r = codes (4h+r, 4h+r+8)
        return 16 * (lb >> 1) + 4 * (lb & 1) + r + 8 * odd;
    }
    if (tier == 1) {  // int4: register r = codes (r, r+4)
        return 8 * lb + r + 4 * odd;
    }
    if (tier == 2) {  // int8 words 2lb, 2lb+1: register r = bytes ((r&1), (r&1)+2) of word 2lb + r/2
        return 4 * (2 * lb + (r >> 1)) + (r & 1) + 2 * odd;
    }
    return 8 * lb + pos;  // fp16: natural order
}

// Exact fp16 integers from magic-exponent patterns 0x6400|code (value 1024 + code).
__device__ __forceinline__ uint32_t unbias(uint32_t x) {
    half2v h = __builtin_bit_cast(half2v, x);
    const half2v b = {static_cast<_Float16>(-1024.0f), static_cast<_Float16>(-1024.0f)};
    return __builtin_bit_cast(uint32_t, h + b);
}

// The 8 fp16 codes of local block ``lb`` of ``tier`` for token row ``tok`` (A operand).
__device__ __forceinline__ half8 load_block(const unsigned char* pb, const MfmaLayout& y, const lf_packed_layer& L,
                                            int tier, int lb, int tok) {
    uint32_t r0 = 0, r1 = 0, r2 = 0, r3 = 0;
    if (lb < y.nblk[tier]) {
        if (tier == 0) {
            const uint32_t w = lds_u32(pb, y.pb_kt[0] + 4 * (tok * L.k_words[0] + (lb >> 1)));
            const uint32_t x = w >> (8 * (lb & 1));
            r0 = unbias((x & 0x00030003u) | 0x64006400u);
            r1 = unbias(((x >> 2) & 0x00030003u) | 0x64006400u);
            r2 = unbias(((x >> 4) & 0x00030003u) | 0x64006400u);
            r3 = unbias(((x >> 6) & 0x00030003u) | 0x64006400u);
        } else if (tier == 1) {
            const uint32_t w = lds_u32(pb, y.pb_kt[1] + 4 * (tok * L.k_words[1] + lb));
            r0 = unbias((w & 0x000F000Fu) | 0x64006400u);
            r1 = unbias(((w >> 4) & 0x000F000Fu) | 0x64006400u);
            r2 = unbias(((w >> 8) & 0x000F000Fu) | 0x64006400u);
            r3 = unbias(((w >> 12) & 0x000F000Fu) | 0x64006400u);
        } else if (tier == 2) {
            const int wi = 2 * lb;
            const uint32_t w0 = lds_u32(pb, y.pb_kt[2] + 4 * (tok * L.k_words[2] + wi));
            const uint32_t w1 = (wi + 1 < L.k_words[2]) ? lds_u32(pb, y.pb_kt[2] + 4 * (tok * L.k_words[2] + wi + 1)) : 0u;
            // bytes (0,2) and (1,3) of each word under a 0x64 high byte
            r0 = unbias(__builtin_amdgcn_perm(w0, 0x64646464u, 0x00060004u));
            r1 = unbias(__builtin_amdgcn_perm(w0, 0x64646464u, 0x00070005u));
            r2 = unbias(__builtin_amdgcn_perm(w1, 0x64646464u, 0x00060004u));
            r3 = unbias(__builtin_amdgcn_perm(w1, 0x64646464u, 0x00070005u));
        } else {
            const uint4 v = *reinterpret_cast<const uint4*>(pb + y.pb_v16 + 2 * (tok * y.w16p + 8 * lb));
            r0 = v.x; r1 = v.y; r2 = v.z; r3 = v.w;
        }
    }
    const uint4 u = {r0, r1, r2, r3};
    return __builtin_bit_cast(half8, u);
}

// 4x4 byte transpose: out[k] = (a0.byte k, a1.byte k, a2.byte k, a3.byte k).
__device__ __forceinline__ void byte_transpose4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t* o) {
    const uint32_t t01_lo = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
    const uint32_t t01_hi = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
    const uint32_t t23_lo = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
    const uint32_t t23_hi = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
    o[0] = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x07060302u);
}

constexpr int kMaxSlots = 2;  // integer-tier slots per thread (nb_int * 8 <= 512)

struct Stage {
    uint4 c[kMaxStage];
    uint32_t v[4];
    uint32_t ks[kMaxSlots];  // fp16 (min << 16 | scale) of the thread's Key slots
    int64_t row0;
};

// Tier and tier-local rank of integer-tier slot ``e`` = 8 * block + position.
__device__ __forceinline__ void slot_of(const MfmaLayout& y, int e, int& tier, int& j) {
    const int gb = e >> 3, pos = e & 7;
    tier = gb >= 4 * y.kfirst[2] ? 2 : gb >= 4 * y.kfirst[1] ? 1 : 0;
    const int lb = gb - 4 * y.kfirst[tier];
    j = lb < y.nblk[tier] ? block_slot(tier, lb, pos) : 0x7fff;
}

// 16-byte chunk ``c`` of page ``row0``'s contiguous blocks (K tiers 0..2, fp16 tier, v scale, v min).
__device__ __forceinline__ uint4 chunk_load(const lf_packed_layer& L, const MfmaLayout& y, int64_t row0, int c) {
    const unsigned char* src;
    int off;
    if (c < y.seg_end[0]) { src = reinterpret_cast<const unsigned char*>(L.k_code[0] + row0 * L.k_words[0]); off = c; }
    else if (c < y.seg_end[1]) { src = reinterpret_cast<const unsigned char*>(L.k_code[1] + row0 * L.k_words[1]); off = c - y.seg_end[0]; }
    else if (c < y.seg_end[2]) { src = reinterpret_cast<const unsigned char*>(L.k_code[2] + row0 * L.k_words[2]); off = c - y.seg_end[1]; }
    else if (c < y.seg_end[3]) { src = reinterpret_cast<const unsigned char*>(L.k_value16 + row0 * L.k_width[3]); off = c - y.seg_end[2]; }
    else if (c < y.seg_end[4]) { src = reinterpret_cast<const unsigned char*>(L.v_scale + row0); off = c - y.seg_end[3]; }
    else { src = reinterpret_cast<const unsigned char*>(L.v_min + row0); off = c - y.seg_end[4]; }
    return *reinterpret_cast<const uint4*>(src + 16 * static_cast<int64_t>(off));
}

// Issue the global loads of page ``page`` of (b, h) into registers (the first kMaxStage
// chunks per thread; stage_store fetches any remainder itself).
__device__ __forceinline__ void stage_load(Stage& s, const lf_packed_layer& L, const MfmaLayout& y, int b, int h,
                                           int page) {
    const int64_t row0 = tok_row(L, b, h, static_cast<int64_t>(page) * kPage);
    s.row0 = row0;
#pragma unroll
    for (int i = 0; i < kMaxStage; ++i) {
        const int c = threadIdx.x + i * kThreads;
        s.c[i] = c < y.seg_end[5] ? chunk_load(L, y, row0, c) : uint4{0u, 0u, 0u, 0u};
    }
    // Value codes: 4 consecutive tokens of one word (token group tid/8, word tid%8).
    const int tg = threadIdx.x >> 3, w = threadIdx.x & 7;
    const int32_t* vc = L.v_code + (row0 + 4 * tg) * 8 + w;
#pragma unroll
    for (int i = 0; i < 4; ++i) s.v[i] = static_cast<uint32_t>(vc[8 * i]);
    // Key scale/min of this page for the thread's integer-tier slots.
#pragma unroll
    for (int i = 0; i < kMaxSlots; ++i) {
        const int e = threadIdx.x + i * kThreads;
        uint32_t v = 0u;
        if (e < y.nb_int * 8) {
            int tier, j;
            slot_of(y, e, tier, j);
            if (j < L.k_width[tier]) {
                const int64_t gi = kgrp_idx(L, b, h, L.k_width[tier], j, page);
                v = static_cast<uint32_t>(L.k_scale[tier][gi]) | (static_cast<uint32_t>(L.k_min[tier][gi]) << 16);
            }
        }
        s.ks[i] = v;
    }
}

// Write one 16-byte chunk into page buffer ``pb``.
__device__ __forceinline__ void chunk_store(unsigned char* pb, const lf_packed_layer& L, const MfmaLayout& y, int c,
                                            uint4 v) {
    if (c < y.seg_end[0]) {
        *reinterpret_cast<uint4*>(pb + y.pb_kt[0] + 16 * c) = v;
    } else if (c < y.seg_end[1]) {
        *reinterpret_cast<uint4*>(pb + y.pb_kt[1] + 16 * (c - y.seg_end[0])) = v;
    } else if (c < y.seg_end[2]) {
        *reinterpret_cast<uint4*>(pb + y.pb_kt[2] + 16 * (c - y.seg_end[1])) = v;
    } else if (c < y.seg_end[3]) {
        // 8 fp16 values of the [128][w16] block -> padded rows [128][w16p]
        const int e0 = 8 * (c - y.seg_end[2]);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint16_t* dst = reinterpret_cast<uint16_t*>(pb + y.pb_v16);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int e = e0 + k;
            const int tok = e / L.k_width[3], j = e - tok * L.k_width[3];
            dst[tok * y.w16p + j] = static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1)));
        }
    } else {
        const bool is_min = c >= y.seg_end[4];
        const int t0 = 8 * (c - (is_min ? y.seg_end[4] : y.seg_end[3]));
        float* dst = reinterpret_cast<float*>(pb + (is_min ? y.pb_vmn : y.pb_vsc)) + t0;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) dst[k] = f16_to_f32(static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1))));
    }
}

// Write staged registers into page buffer ``pb``; chunks past the register budget are
// fetched here directly.
__device__ __forceinline__ void stage_store(const Stage& s, unsigned char* pb, const lf_packed_layer& L,
                                            const MfmaLayout& y) {
#pragma unroll
    for (int i = 0; i < kMaxStage; ++i) {
        const int c = threadIdx.x + i * kThreads;
        if (c < y.seg_end[5]) chunk_store(pb, L, y, c, s.c[i]);
    }
    for (int c = threadIdx.x + kMaxStage * kThreads; c < y.seg_end[5]; c += kThreads)
        chunk_store(pb, L, y, c, chunk_load(L, y, s.row0, c));
#pragma unroll
    for (int i = 0; i < kMaxSlots; ++i) {
        const int e = threadIdx.x + i * kThreads;
        if (e < y.nb_int * 8) {
            reinterpret_cast<float*>(pb + y.pb_ksc)[e] = f16_to_f32(static_cast<uint16_t>(s.ks[i] & 0xffffu));
            reinterpret_cast<float*>(pb + y.pb_kmn)[e] = f16_to_f32(static_cast<uint16_t>(s.ks[i] >> 16));
        }
    }
    uint32_t o[4];
    byte_transpose4(s.v[0], s.v[1], s.v[2], s.v[3], o);
    const int tg = threadIdx.x >> 3, w = threadIdx.x & 7;
    uint32_t* vt = reinterpret_cast<uint32_t*>(pb + y.pb_vt);
#pragma unroll
    for (int k = 0; k < 4; ++k) vt[(tg * 4 + k) * 8 + w] = o[k];
}

__global__ __launch_bounds__(kThreads, 2) void decode_mfma_kernel(MfmaParams mp) {
    const DecodeParams& p = mp.p;
    const MfmaLayout& y = mp.y;
    const lf_packed_layer& L = p.L;
    const lf_decode_args& A = p.A;
    const int item = blockIdx.x;
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n16 = lane & 15;   // MFMA column / row index
    const int kb = lane >> 4;    // lane group
    const int g = p.g;
    const int b = A.work[4 * item + 0];
    const int pbeg = A.work[4 * item + 1];
    const int pend = A.work[4 * item + 2];
    const int kind = A.work[4 * item + 3];

    extern __shared__ __align__(16) unsigned char smem[];
    float* qperm = reinterpret_cast<float*>(smem + y.off_qperm);
    float* small = reinterpret_cast<float*>(smem + y.off_small);
    float* bpart = small;                 // [4 waves][8]: partial bias sums
    float* alpha_lds = small + 32;        // [4 waves][8]: softmax rescale per head
    float* wstat = small + 64;            // [4 waves][3][8]: m, l, mv per head
    float* qlin = reinterpret_cast<float*>(smem + y.off_pb[0]);  // [8][128] q (residual path only)

    // ---- q (scaled into the log2 domain) and this head's tier table, one coalesced pass ----
    int16_t* tt = reinterpret_cast<int16_t*>(smem + y.off_tt);  // ranks -> channels, tiers back to back
    int tt_off[4];
    tt_off[0] = 0;
    for (int t = 1; t < 4; ++t) tt_off[t] = tt_off[t - 1] + L.k_width[t - 1];
    for (int e = tid; e < 8 * kD; e += kThreads) {
        const int n = e / kD, c = e % kD;
        qlin[e] = n < g ? load_as_f32(A.query, (static_cast<int64_t>(b) * A.n_q + h * g + n) * kD + c, A.q_dtype) *
                              p.qscale
                        : 0.f;
    }
    for (int e = tid; e < tt_off[3] + L.k_width[3]; e += kThreads) {
        const int t = e >= tt_off[3] ? 3 : e >= tt_off[2] ? 2 : e >= tt_off[1] ? 1 : 0;
        const int j = e - tt_off[t];
        tt[e] = j < L.tier_count[t][h] ? static_cast<int16_t>(L.tier_index[t][h * L.k_width[t] + j]) : int16_t(-1);
    }
    __syncthreads();
    // q permuted into slot order (0 for padding slots and heads >= g)
    for (int e = tid; e < y.nb * 64; e += kThreads) {
        const int gb = e >> 6, n = (e >> 3) & 7, pos = e & 7;
        int tier = 3;
        for (int t = 0; t < 3; ++t)
            if (gb < 4 * (y.kfirst[t] + y.kst[t])) { tier = t; break; }
        const int lb = gb - 4 * y.kfirst[tier];
        float v = 0.f;
        if (lb < y.nblk[tier]) {
            const int j = block_slot(tier, lb, pos);
            if (j < L.k_width[tier]) {
                const int c = tt[tt_off[tier] + j];
                if (c >= 0) v = qlin[n * kD + c];
            }
        }
        qperm[e] = v;
    }
    __syncthreads();

    float O[8][4];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[nt][r] = 0.f;
    float m_run = -__builtin_inff(), l_run = 0.f, mv_run = 0.f;

    if (kind == 0) {
        // fp16-tier rows are padded to w16p columns; the padding must read as zero
        for (int e = tid; e < kPage * y.w16p / 2; e += kThreads) {
            reinterpret_cast<uint32_t*>(smem + y.off_pb[0] + y.pb_v16)[e] = 0u;
            reinterpret_cast<uint32_t*>(smem + y.off_pb[1] + y.pb_v16)[e] = 0u;
        }
        __syncthreads();
        Stage st;
        stage_load(st, L, y, b, h, pbeg);
        stage_store(st, smem + y.off_pb[0], L, y);
        __syncthreads();
        half8* qs = reinterpret_cast<half8*>(smem + y.off_qs);
        for (int page = pbeg; page < pend; ++page) {
            const int rel = page - pbeg;
            const int cbuf = rel & 1;
            unsigned char* pb = smem + y.off_pb[cbuf];
            const float* sc = reinterpret_cast<const float*>(pb + y.pb_ksc);
            const float* mn = reinterpret_cast<const float*>(pb + y.pb_kmn);
            // Prefetch the next page into registers.
            const bool more = page + 1 < pend;
            if (more) stage_load(st, L, y, b, h, page + 1);
            // Qs (hi rows 0..7, lo rows 8..15) for this page.
            for (int e = tid; e < y.nb * 16; e += kThreads) {
                const int gb = e >> 4, row = e & 15, n = row & 7;
                const float* qrow = qperm + (gb * 8 + n) * 8;
                float qv[8];
                if (gb < y.nb_int) {
                    const float* srow = sc + gb * 8;
#pragma unroll
                    for (int k = 0; k < 8; ++k) qv[k] = qrow[k] * srow[k];
                } else {
#pragma unroll
                    for (int k = 0; k < 8; ++k) qv[k] = qrow[k];
                }
                half8 hv;
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const _Float16 hi = static_cast<_Float16>(qv[k]);
                    hv[k] = row < 8 ? hi : static_cast<_Float16>(qv[k] - static_cast<float>(hi));
                }
                qs[e] = hv;
            }
            // bias[n] = sum over integer-tier slots of q * min
            {
                const int n = tid & 7, part = tid >> 3;  // 32 parts
                float acc = 0.f;
                for (int gb = part; gb < y.nb_int; gb += 32) {
                    const float* qrow = qperm + (gb * 8 + n) * 8;
                    const float* mrow = mn + gb * 8;
#pragma unroll
                    for (int k = 0; k < 8; ++k) acc = fmaf(qrow[k], mrow[k], acc);
                }
                acc += __shfl_xor(acc, 8, kWave);
                acc += __shfl_xor(acc, 16, kWave);
                acc += __shfl_xor(acc, 32, kWave);
                if (lane < 8) bpart[wave * 8 + lane] = acc;
            }
            __syncthreads();
            const float bias = (n16 < 8) ? bpart[n16] + bpart[8 + n16] + bpart[16 + n16] + bpart[24 + n16] : 0.f;

            // ---- scores for this wave's 32 tokens ----
            float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
            const int tok0 = 32 * wave + n16, tok1 = tok0 + 16;
            for (int t = 0; t < 4; ++t) {
                for (int s = 0; s < y.kst[t]; ++s) {
                    const int gks = y.kfirst[t] + s;
                    const half8 bq = qs[(4 * gks + kb) * 16 + n16];
                    const int lb = 4 * s + kb;
                    const half8 a0 = load_block(pb, y, L, t, lb, tok0);
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, bq, acc0, 0, 0, 0);
                    const half8 a1 = load_block(pb, y, L, t, lb, tok1);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, bq, acc1, 0, 0, 0);
                }
            }
            // hi + lo columns, + bias; lanes n16 >= 8 carry don't-care values.  The accumulator
            // elements are copied to scalars before the DPP move: applied directly to vector
            // elements, this compiler emits a single DPP move for all of them.
            float sv[8];
            const float accs[8] = {acc0[0], acc0[1], acc0[2], acc0[3], acc1[0], acc1[1], acc1[2], acc1[3]};
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int xi = __builtin_bit_cast(int, accs[r]);
                sv[r] = accs[r] + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(xi, xi, 0x108, 0xf, 0xf, false)) +
                        bias;
            }
            // ---- online softmax (log2 domain) ----
            float mx = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sv[i]);
            mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
            mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            m_run = m_new;
            const float* vsc = reinterpret_cast<const float*>(pb + y.pb_vsc);
            const float* vmn = reinterpret_cast<const float*>(pb + y.pb_vmn);
            const float4 s_lo = *reinterpret_cast<const float4*>(vsc + 32 * wave + 4 * kb);
            const float4 s_hi = *reinterpret_cast<const float4*>(vsc + 32 * wave + 16 + 4 * kb);
            const float4 m_lo = *reinterpret_cast<const float4*>(vmn + 32 * wave + 4 * kb);
            const float4 m_hi = *reinterpret_cast<const float4*>(vmn + 32 * wave + 16 + 4 * kb);
            const float vs[8] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w, s_hi.x, s_hi.y, s_hi.z, s_hi.w};
            const float vm[8] = {m_lo.x, m_lo.y, m_lo.z, m_lo.w, m_hi.x, m_hi.y, m_hi.z, m_hi.w};
            float pp[8];
            float psum = 0.f, pmin = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pi = __builtin_amdgcn_exp2f(sv[i] - m_new);
                psum += pi;
                pmin = fmaf(pi, vm[i], pmin);
                pp[i] = pi * vs[i];
            }
            l_run = l_run * alpha + psum;
            mv_run = mv_run * alpha + pmin;
            // A operand of the value product: k order (t0,t2),(t1,t3),(t4,t6),(t5,t7) of the lane's
            // tokens; hi in lanes n16 < 8, lo (moved 8 lanes up) in lanes n16 >= 8.
            uint32_t ahi[4], alo[4];
            const int order[8] = {0, 2, 1, 3, 4, 6, 5, 7};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float x0 = pp[order[2 * j]], x1 = pp[order[2 * j + 1]];
                const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
                const half2v hv = {h0, h1};
                const half2v lv = {static_cast<_Float16>(x0 - static_cast<float>(h0)),
                                   static_cast<_Float16>(x1 - static_cast<float>(h1))};
                ahi[j] = __builtin_bit_cast(uint32_t, hv);
                alo[j] = __builtin_bit_cast(uint32_t, lv);
            }
            uint4 au;
            au.x = __builtin_amdgcn_update_dpp(ahi[0], alo[0], 0x118, 0xf, 0xc, false);
            au.y = __builtin_amdgcn_update_dpp(ahi[1], alo[1], 0x118, 0xf, 0xc, false);
            au.z = __builtin_amdgcn_update_dpp(ahi[2], alo[2], 0x118, 0xf, 0xc, false);
            au.w = __builtin_amdgcn_update_dpp(ahi[3], alo[3], 0x118, 0xf, 0xc, false);
            const half8 ap = __builtin_bit_cast(half8, au);
            // alpha of the 4 output rows this lane holds (rows 4*kb + r, head (4*kb + r) % 8)
            // (same-wave LDS write then read: ordered by the LDS queue)
            if (kb == 0 && n16 < 8) alpha_lds[wave * 8 + n16] = alpha;
            __builtin_amdgcn_wave_barrier();
            const float4 arow = *reinterpret_cast<const float4*>(alpha_lds + wave * 8 + 4 * (kb & 1));
            // ---- value product ----
            const uint32_t* vt = reinterpret_cast<const uint32_t*>(pb + y.pb_vt);
            const uint4 d0a = *reinterpret_cast<const uint4*>(vt + ((8 * wave + kb) * 4 + (n16 >> 2)) * 8);
            const uint4 d0b = *reinterpret_cast<const uint4*>(vt + ((8 * wave + kb) * 4 + (n16 >> 2)) * 8 + 4);
            const uint4 d1a = *reinterpret_cast<const uint4*>(vt + ((8 * wave + 4 + kb) * 4 + (n16 >> 2)) * 8);
            const uint4 d1b = *reinterpret_cast<const uint4*>(vt + ((8 * wave + 4 + kb) * 4 + (n16 >> 2)) * 8 + 4);
            const uint32_t dlo[8] = {d0a.x, d0a.y, d0a.z, d0a.w, d0b.x, d0b.y, d0b.z, d0b.w};
            const uint32_t dhi[8] = {d1a.x, d1a.y, d1a.z, d1a.w, d1b.x, d1b.y, d1b.z, d1b.w};
            const int sh = 2 * (n16 & 3);
            const half2v inv256 = {static_cast<_Float16>(1.0f / 256.0f), static_cast<_Float16>(1.0f / 256.0f)};
            const half2v m4 = {static_cast<_Float16>(-4.0f), static_cast<_Float16>(-4.0f)};
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                const uint32_t xl = dlo[nt] >> sh, xh = dhi[nt] >> sh;
                uint4 bu;
                bu.x = unbias((xl & 0x00030003u) | 0x64006400u);                     // tokens (0, 2)
                bu.y = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, (xl & 0x03000300u) | 0x64006400u) * inv256 + m4);  // (1, 3)
                bu.z = unbias((xh & 0x00030003u) | 0x64006400u);
                bu.w = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, (xh & 0x03000300u) | 0x64006400u) * inv256 + m4);
                const half8 bv = __builtin_bit_cast(half8, bu);
                float4v o4 = {O[nt][0] * arow.x, O[nt][1] * arow.y, O[nt][2] * arow.z, O[nt][3] * arow.w};
                o4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap, bv, o4, 0, 0, 0);
                O[nt][0] = o4[0]; O[nt][1] = o4[1]; O[nt][2] = o4[2]; O[nt][3] = o4[3];
            }
            // Publish the prefetched page into the other buffer; the barrier also retires this page.
            if (more) stage_store(st, smem + y.off_pb[cbuf ^ 1], L, y);
            __syncthreads();
        }
        // Reduce l and the value-minimum term over the 4 lane groups of each head.
        l_run += __shfl_xor(l_run, 16, kWave);
        l_run += __shfl_xor(l_run, 32, kWave);
        mv_run += __shfl_xor(mv_run, 16, kWave);
        mv_run += __shfl_xor(mv_run, 32, kWave);
        // Rows r (hi, lanes kb 0..1) + rows r+8 (lo, lanes kb 2..3).
#pragma unroll
        for (int nt = 0; nt < 8; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) O[nt][r] += __shfl_xor(O[nt][r], 32, kWave);
    } else {
        // ---- residual item: the tail page and the new token (at most page_size tokens) ----
        // VALU: wave w scores tokens 32w..32w+31 (lane = token), then accumulates them into
        // channels 2*lane, 2*lane+1.  One pass, so each wave's max is final.
        for (int e = tid; e < 8 * kD; e += kThreads) {
            const int n = e / kD, c = e % kD;
            qlin[e] = n < g ? load_as_f32(A.query, (static_cast<int64_t>(b) * A.n_q + h * g + n) * kD + c, A.q_dtype) *
                                  p.qscale
                            : 0.f;
        }
        __syncthreads();
        const int tl = A.tail_len[b];
        const int n_res = tl + (A.k_new != nullptr ? 1 : 0);
        const int t = 32 * wave + lane;
        const bool act = lane < 32 && t < n_res;
        float s[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] = 0.f;
        if (act) {
            const void* kp = t < tl ? A.tail_k : A.k_new;
            const int kdt = t < tl ? A.tail_dtype : A.new_dtype;
            const int64_t kbase = t < tl ? ((static_cast<int64_t>(b) * L.n_kv + h) * A.tail_cap + t) * kD
                                         : (static_cast<int64_t>(b) * L.n_kv + h) * kD;
            for (int c0 = 0; c0 < kD; c0 += 32) {
                float kv[4][8];
#pragma unroll
                for (int u = 0; u < 4; ++u) load8_as_f32(kp, kbase + c0 + 8 * u, kdt, kv[u]);
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int k = 0; k < 8; ++k)
#pragma unroll
                        for (int i = 0; i < 8; ++i) s[i] = fmaf(qlin[i * kD + c0 + 8 * u + k], kv[u][k], s[i]);
            }
        }
        float* pbuf = reinterpret_cast<float*>(smem + y.off_pbuf) + wave * 32 * 8;  // [32][8]
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = act ? s[i] : -__builtin_inff();
            const float mx = wave_max(x);
            const float pi = act ? __builtin_amdgcn_exp2f(x - mx) : 0.f;
            const float lt = wave_sum(pi);
            if (lane < 32) pbuf[lane * 8 + i] = pi;
            if (lane == 0) {
                wstat[(wave * 3 + 0) * 8 + i] = mx;
                wstat[(wave * 3 + 1) * 8 + i] = lt;
                wstat[(wave * 3 + 2) * 8 + i] = 0.f;
            }
        }
        __builtin_amdgcn_wave_barrier();
        const int cnt = max(0, min(32, n_res - 32 * wave));
        float acc[2][8];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[cc][i] = 0.f;
        const int64_t vrow0 = ((static_cast<int64_t>(b) * L.n_kv + h) * A.tail_cap) * kD;
        const int64_t vnew = (static_cast<int64_t>(b) * L.n_kv + h) * kD;
#pragma unroll 8
        for (int tt = 0; tt < cnt; ++tt) {
            const int tok = 32 * wave + tt;
            float v0, v1;
            if (tok < tl) {
                v0 = load_as_f32(A.tail_v, vrow0 + static_cast<int64_t>(tok) * kD + 2 * lane, A.tail_dtype);
                v1 = load_as_f32(A.tail_v, vrow0 + static_cast<int64_t>(tok) * kD + 2 * lane + 1, A.tail_dtype);
            } else {
                v0 = load_as_f32(A.v_new, vnew + 2 * lane, A.new_dtype);
                v1 = load_as_f32(A.v_new, vnew + 2 * lane + 1, A.new_dtype);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                acc[0][i] = fmaf(pbuf[tt * 8 + i], v0, acc[0][i]);
                acc[1][i] = fmaf(pbuf[tt * 8 + i], v1, acc[1][i]);
            }
        }
        float* red = reinterpret_cast<float*>(smem + y.off_pb[0]) + 8 * kD;  // [4][8][128], after qlin
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int i = 0; i < 8; ++i) red[(wave * 8 + i) * kD + 2 * lane + cc] = acc[cc][i];
        __syncthreads();
    }

    // ---- merge the 4 waves and store this item's partial ----
    float* red = reinterpret_cast<float*>(smem + y.off_pb[0]) + 8 * kD;  // [4][8][128]
    if (kind == 0) {
        __syncthreads();
        // head rows held by lanes kb 0..1: row 4*kb + r, channel 16*nt + n16
        if (kb < 2) {
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[(wave * 8 + 4 * kb + r) * kD + 16 * nt + n16] = O[nt][r];
        }
        if (kb == 0 && n16 < 8) {
            wstat[(wave * 3 + 0) * 8 + n16] = m_run;
            wstat[(wave * 3 + 1) * 8 + n16] = l_run;
            wstat[(wave * 3 + 2) * 8 + n16] = mv_run;
        }
        __syncthreads();
    }
    for (int e = tid; e < g * kD; e += kThreads) {
        const int i = e / kD, c = e % kD;
        float M = -__builtin_inff();
        for (int w = 0; w < 4; ++w) M = fmaxf(M, wstat[(w * 3 + 0) * 8 + i]);
        float o = 0.f, l = 0.f;
        if (M != -__builtin_inff()) {
            for (int w = 0; w < 4; ++w) {
                const float mw = wstat[(w * 3 + 0) * 8 + i];
                const float sc = __builtin_amdgcn_exp2f(mw - M);
                o += sc * (red[(w * 8 + i) * kD + c] + wstat[(w * 3 + 2) * 8 + i]);
                l += sc * wstat[(w * 3 + 1) * 8 + i];
            }
        }
        float* rec = part_rec(p, item, h, i);
        rec[c] = o;
        if (c == 0) {
            rec[kD] = M;
            rec[kD + 1] = l;
        }
    }
    __shared__ int flag;
    if (last_split_arrives(p, b, h, &flag))
        merge_partials(p, b, h, reinterpret_cast<float*>(smem + y.off_merge), y.merge_floats);
}

int round_up(int x, int m) { return (x + m - 1) / m * m; }

// Host: LDS layout for this layer; false when the shape is outside this kernel.
bool plan_layout(const lf_packed_layer& L, int g, MfmaLayout& y) {
    if (L.head_dim != kD || L.page_size != kPage || L.k_group != kPage || L.bit_v != 2 || L.v_group != kD)
        return false;
    if (g < 1 || g > 8) return false;
    y.nblk[0] = 2 * L.k_words[0];
    y.nblk[1] = L.k_words[1];
    y.nblk[2] = (L.k_words[2] + 1) / 2;
    y.nblk[3] = (L.k_width[3] + 7) / 8;
    int ks = 0;
    for (int t = 0; t < 4; ++t) {
        y.kst[t] = (y.nblk[t] + 3) / 4;
        y.kfirst[t] = ks;
        ks += y.kst[t];
    }
    y.nb = 4 * ks;
    y.nb_int = 4 * (y.kst[0] + y.kst[1] + y.kst[2]);
    y.w16p = round_up(L.k_width[3], 8);
    int off = 0;
    y.off_qperm = off; off += y.nb * 64 * 4;
    y.off_qs = off; off += y.nb * 16 * 16;
    y.off_merge = 0;
    y.merge_floats = off / 4;
    y.off_tt = off; off += round_up(2 * (L.k_width[0] + L.k_width[1] + L.k_width[2] + L.k_width[3]), 16);
    y.off_small = off; off += (32 + 32 + 96) * 4;
    y.off_pbuf = off; off += 4 * 32 * 8 * 4;
    off = round_up(off, 16);
    int pb = 0;
    for (int t = 0; t < 3; ++t) { y.pb_kt[t] = pb; pb += kPage * L.k_words[t] * 4; }
    y.pb_v16 = pb; pb += kPage * y.w16p * 2;
    pb = round_up(pb, 16);
    y.pb_vt = pb; pb += 32 * 4 * 8 * 4;
    y.pb_vsc = pb; pb += kPage * 4;
    y.pb_vmn = pb; pb += kPage * 4;
    y.pb_ksc = pb; pb += y.nb_int * 8 * 4;
    y.pb_kmn = pb; pb += y.nb_int * 8 * 4;
    pb = round_up(pb, 16);
    // the reduction area [8][128] q + [4][8][128] wave outputs aliases the page buffers
    const int red_bytes = (8 + 32) * kD * 4;
    if (2 * pb < red_bytes) pb = round_up(red_bytes, 32) / 2;
    y.off_pb[0] = off;
    y.off_pb[1] = off + pb;
    off += 2 * pb;
    y.lds_bytes = off;
    int seg = 0;
    for (int t = 0; t < 3; ++t) { seg += kPage * L.k_words[t] * 4 / 16; y.seg_end[t] = seg; }
    seg += kPage * L.k_width[3] * 2 / 16; y.seg_end[3] = seg;
    seg += kPage * 2 / 16; y.seg_end[4] = seg;
    seg += kPage * 2 / 16; y.seg_end[5] = seg;
    if (y.nb_int * 8 > kMaxSlots * kThreads) return false;
    if (y.lds_bytes > 160 * 1024 - 64) return false;
    return true;
}

}  // namespace

int launch_decode_mfma(const DecodeParams& p, hipStream_t stream, bool* handled) {
    MfmaParams mp;
    mp.p = p;
    if (!plan_layout(p.L, p.g, mp.y)) {
        *handled = false;
        return LF_OK;
    }
    *handled = true;
    // Raise the dynamic-LDS limit to what this launch needs (static LDS counts against the same budget).
    static int lds_limit = 64 * 1024;
    if (mp.y.lds_bytes > lds_limit) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&decode_mfma_kernel),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, mp.y.lds_bytes);
        if (e != hipSuccess) return static_cast<int>(e);
        lds_limit = mp.y.lds_bytes;
    }
    hipLaunchKernelGGL(decode_mfma_kernel, dim3(p.A.n_work, p.L.n_kv), dim3(kThreads), mp.y.lds_bytes, stream, mp);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
