// Page compress: one 128-token (page_size) BF16 page per (sequence, kv head)
// -> the reference's packed byte layout.
//
// Reference: src/logitfill/packed/layout.py:12-35 (asymmetric_codes, pack_ints),
// :71-112 (quantize_key_page), :115-129 (quantize_value_page), written at the
// page's offset of the history (src/logitfill/packed/cache.py:64-81).
//
// Numerics are those of the reference's float32 torch CPU arithmetic:
//   lo = min, hi = max over the group; s = clamp((hi - lo) / qmax, 1e-5, 1e5)
//   with IEEE division; code = clamp(rint_half_even((x - lo) / s), 0, qmax);
//   scale/min stored as float16 (round to nearest even).
// This translation unit is compiled without FP contraction so that every
// subtraction and division is a separately rounded IEEE operation.
//
// One workgroup (256 threads) packs one page of one kv head: the page is
// staged in LDS; Key groups run down channels (two threads per channel and
// token group), Value groups along each token (two threads per token and
// channel group); 8-bit codes are collected in LDS and assembled into
// LSB-first int32 words written with coalesced stores.
#pragma clang fp contract(off)

#include "lf_common.hpp"

namespace lf {
namespace {

constexpr int kPackThreads = 256;

struct PackJobArgs {
    lf_packed_layer L;
    const void* k_src;
    const void* v_src;
    int64_t sb, sh, st;
    const int32_t* jobs;
    int vec16;  // 1 when every page row is 16-byte aligned
    int cw;     // bytes per LDS code row: max(head_dim, sum of int tier widths)
};

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t x) { return bf16_to_f32(x); }
template <>
__device__ __forceinline__ float to_f32<float>(float x) { return x; }


template <typename T, bool IsHalf>
__device__ __forceinline__ float elem_f32(T x) {
    if constexpr (IsHalf) return f16_to_f32(x);
    else return to_f32<T>(x);
}

// Stage a [P][D] page (row stride ``ld`` elements in LDS) from global memory.
template <typename T>
__device__ void stage_page(T* lds, int ld, const T* src, int64_t st, int P, int D, bool vec16) {
    constexpr int kPer16 = 16 / sizeof(T);
    if (vec16 && (D % kPer16) == 0) {
        const int chunks = D / kPer16;
        for (int idx = threadIdx.x; idx < P * chunks; idx += kPackThreads) {
            const int row = idx / chunks;
            const int col = (idx % chunks) * kPer16;
            const uint4 v = *reinterpret_cast<const uint4*>(src + row * st + col);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
            uint32_t* dst = reinterpret_cast<uint32_t*>(lds + row * ld + col);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = w[i];
        }
    } else {
        for (int idx = threadIdx.x; idx < P * D; idx += kPackThreads) {
            const int row = idx / D;
            const int col = idx % D;
            lds[row * ld + col] = src[row * st + col];
        }
    }
}

// s = clamp((hi - lo) / qmax, 1e-5, 1e5) in float32 (layout.py:16).
__device__ __forceinline__ float group_scale(float hi, float lo, int qmax) {
    const float s = (hi - lo) / static_cast<float>(qmax);
    return fminf(fmaxf(s, 1e-5f), 1e5f);
}

// code = clamp(round_half_even((x - lo) / s), 0, qmax) (layout.py:17).
__device__ __forceinline__ uint32_t group_code(float x, float lo, float s, int qmax) {
    const float q = __builtin_rintf((x - lo) / s);
    return static_cast<uint32_t>(fminf(fmaxf(q, 0.0f), static_cast<float>(qmax)));
}

// ``Staged``: the page is copied to LDS first; otherwise (pages too large for LDS next to the
// code rows) every element is read from global memory where it is used.
template <typename T, bool IsHalf, bool Staged>
__global__ __launch_bounds__(kPackThreads) void pack_pages_kernel(PackJobArgs a) {
    const lf_packed_layer& L = a.L;
    const int job = blockIdx.x;
    const int h = blockIdx.y;
    const int b = a.jobs[3 * job + 0];
    const int64_t tok0 = a.jobs[3 * job + 1];
    const int page = a.jobs[3 * job + 2];
    const int P = L.page_size;
    const int D = L.head_dim;
    const int ld = D + (sizeof(T) == 2 ? 2 : 1);
    const int64_t dst_tok0 = static_cast<int64_t>(page) * P;

    extern __shared__ __align__(16) unsigned char smem[];
    T* page_lds = reinterpret_cast<T*>(smem);
    const int cw = a.cw;
    uint8_t* codes = smem + (Staged ? static_cast<size_t>(P) * ld * sizeof(T) : 0);  // [P][cw]
    int8_t* tier_of = reinterpret_cast<int8_t*>(codes + P * cw);         // [D]
    int16_t* local_of = reinterpret_cast<int16_t*>(tier_of + ((D + 1) & ~1));  // [D]

    // ---- tier map for this head (layout.py:49-68) ----
    for (int c = threadIdx.x; c < D; c += kPackThreads) { tier_of[c] = -1; local_of[c] = -1; }
    for (int i = threadIdx.x; i < P * cw; i += kPackThreads) codes[i] = 0;
    __syncthreads();
    for (int t = 0; t < 4; ++t) {
        if (L.k_width[t] == 0) continue;
        const int cnt = L.tier_count[t][h];
        for (int j = threadIdx.x; j < cnt; j += kPackThreads) {
            const int c = L.tier_index[t][h * L.k_width[t] + j];
            tier_of[c] = static_cast<int8_t>(t);
            local_of[c] = static_cast<int16_t>(j);
        }
    }
    int koff[4];
    koff[0] = 0;
    koff[1] = L.k_width[0];
    koff[2] = koff[1] + L.k_width[1];
    koff[3] = koff[2] + L.k_width[2];

    // ---- Key page ----
    const T* ksrc = static_cast<const T*>(a.k_src) + b * a.sb + h * a.sh + tok0 * a.st;
    const T* vsrc = static_cast<const T*>(a.v_src) + b * a.sb + h * a.sh + tok0 * a.st;
    const T* cur = ksrc;  // the page the accessor below reads
    auto at = [&](int tau, int c) -> T { return Staged ? page_lds[tau * ld + c] : cur[tau * a.st + c]; };
    if (Staged) stage_page<T>(page_lds, ld, ksrc, a.st, P, D, a.vec16 != 0);
    __syncthreads();

    const int kg = L.k_group;
    const int ngroups = P / kg;
    const int64_t grp0 = static_cast<int64_t>(page) * ngroups;
    for (int u0 = 0; u0 < D * ngroups; u0 += kPackThreads / 2) {
        const int u = u0 + (threadIdx.x >> 1);
        const int half = threadIdx.x & 1;
        const bool live = u < D * ngroups;
        const int c = live ? (u % D) : 0;
        const int g = live ? (u / D) : 0;
        const int t0 = live ? tier_of[c] : 3;
        const bool quant = live && t0 >= 0 && t0 < 3;
        const int t = quant ? t0 : 0;
        const int bits = 2 << t;
        const int qmax = (1 << bits) - 1;
        const int beg = g * kg + (half ? kg / 2 : 0);
        const int end = half ? (g + 1) * kg : g * kg + kg / 2;
        float lo = __builtin_inff(), hi = -__builtin_inff();
        if (quant) {
            for (int tau = beg; tau < end; ++tau) {
                const float x = elem_f32<T, IsHalf>(at(tau, c));
                lo = fminf(lo, x);
                hi = fmaxf(hi, x);
            }
        }
        lo = fminf(lo, __shfl_xor(lo, 1, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, 1, kWave));
        if (quant) {
            const float s = group_scale(hi, lo, qmax);
            const int j = local_of[c];
            uint8_t* crow = codes + koff[t] + j;
            for (int tau = beg; tau < end; ++tau) {
                const float x = elem_f32<T, IsHalf>(at(tau, c));
                crow[tau * cw] = static_cast<uint8_t>(group_code(x, lo, s, qmax));
            }
            if (half == 0) {
                const int64_t o = kgrp_idx(L, b, h, L.k_width[t], j, grp0 + g);
                const uint16_t hs = f32_to_f16(s), hl = f32_to_f16(lo);
                L.k_scale[t][o] = hs;
                L.k_min[t][o] = hl;
                if (L.k_sm_page != nullptr && ngroups == 1) {  // the page-major copy (one Key group a page)
                    int lb, bp;
                    sm_place(t, j, lb, bp);
                    uint16_t* blk = L.k_sm_page + sm_page_idx(L, b, h, page) + 16 * (sm_page(L.k_words).blk0[t] + lb);
                    blk[bp] = hs;
                    blk[8 + bp] = hl;
                }
            }
        }
    }
    // Padding slots of each tier keep scale 1.0 and min 0.0 (layout.py:84-85).
    for (int t = 0; t < 3; ++t) {
        const int w = L.k_width[t];
        const int cnt = L.tier_count[t] ? L.tier_count[t][h] : 0;
        for (int idx = threadIdx.x; idx < (w - cnt) * ngroups; idx += kPackThreads) {
            const int j = cnt + idx / ngroups;
            const int g = idx % ngroups;
            const int64_t o = kgrp_idx(L, b, h, w, j, grp0 + g);
            L.k_scale[t][o] = 0x3C00u;
            L.k_min[t][o] = 0;
        }
    }
    // The page-major copy's positions of no channel of this head: scale 1.0, min 0.0.
    if (L.k_sm_page != nullptr && ngroups == 1) {
        const SmPage sp = sm_page(L.k_words);
        for (int p = threadIdx.x; p < 8 * sp.nb; p += kPackThreads) {
            const int gb = p >> 3, pos = p & 7;
            const int t = gb >= sp.blk0[2] ? 2 : gb >= sp.blk0[1] ? 1 : 0;
            const int cnt = L.k_width[t] ? L.tier_count[t][h] : 0;
            if (sm_slot(t, gb - sp.blk0[t], pos) >= cnt) {
                uint16_t* blk = L.k_sm_page + sm_page_idx(L, b, h, page) + 16 * gb;
                blk[pos] = 0x3C00u;
                blk[8 + pos] = 0;
            }
        }
    }
    __syncthreads();

    // Assemble LSB-first words per tier (layout.py:21-35, :94-97).
    for (int t = 0; t < 3; ++t) {
        const int words = L.k_words[t];
        if (words == 0) continue;
        const int bits = 2 << t;
        const int per = 32 / bits;
        const int width = L.k_width[t];
        int32_t* out = L.k_code[t] + tok_row(L, b, h, dst_tok0) * words;
        for (int idx = threadIdx.x; idx < P * words; idx += kPackThreads) {
            const int tau = idx / words;
            const int w = idx % words;
            const uint8_t* crow = codes + tau * cw + koff[t];
            uint32_t word = 0;
            for (int k = 0; k < per; ++k) {
                const int slot = w * per + k;
                if (slot < width) word |= static_cast<uint32_t>(crow[slot]) << (k * bits);
            }
            out[idx] = static_cast<int32_t>(word);
        }
    }
    // fp16 tier: float16 copies of the input values (layout.py:101-111).
    if (L.k_width[3] > 0) {
        const int w16 = L.k_width[3];
        const int cnt = L.tier_count[3][h];
        uint16_t* out = L.k_value16 + tok_row(L, b, h, dst_tok0) * w16;
        for (int idx = threadIdx.x; idx < P * w16; idx += kPackThreads) {
            const int tau = idx / w16;
            const int j = idx % w16;
            uint16_t v = 0;
            if (j < cnt) {
                const int c = L.tier_index[3][h * w16 + j];
                if constexpr (IsHalf) v = static_cast<uint16_t>(at(tau, c));
                else v = f32_to_f16(elem_f32<T, IsHalf>(at(tau, c)));
            }
            out[idx] = v;
        }
    }
    __syncthreads();

    // ---- Value page (layout.py:115-129) ----
    cur = vsrc;
    if (Staged) stage_page<T>(page_lds, ld, vsrc, a.st, P, D, a.vec16 != 0);
    __syncthreads();

    if (L.bit_v >= 16) {
        uint16_t* out = L.v_value16 + tok_row(L, b, h, dst_tok0) * D;
        for (int idx = threadIdx.x; idx < P * D; idx += kPackThreads) {
            const int tau = idx / D;
            const int c = idx % D;
            if constexpr (IsHalf) out[idx] = static_cast<uint16_t>(at(tau, c));
            else out[idx] = f32_to_f16(elem_f32<T, IsHalf>(at(tau, c)));
        }
        return;
    }

    const int vg = L.v_group;
    const int vgroups = L.v_groups;
    const int vbits = L.bit_v;
    const int vqmax = (1 << vbits) - 1;
    for (int u0 = 0; u0 < P * vgroups; u0 += kPackThreads / 2) {
        const int u = u0 + (threadIdx.x >> 1);
        const int half = threadIdx.x & 1;
        const bool live = u < P * vgroups;
        const int tau = live ? u / vgroups : 0;
        const int g = live ? u % vgroups : 0;
        const int beg = g * vg + (half ? vg / 2 : 0);
        const int end = half ? (g + 1) * vg : g * vg + vg / 2;
        float lo = __builtin_inff(), hi = -__builtin_inff();
        if (live) {
            for (int c = beg; c < end; ++c) {
                const float x = elem_f32<T, IsHalf>(at(tau, c));
                lo = fminf(lo, x);
                hi = fmaxf(hi, x);
            }
        }
        lo = fminf(lo, __shfl_xor(lo, 1, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, 1, kWave));
        if (live) {
            const float s = group_scale(hi, lo, vqmax);
            for (int c = beg; c < end; ++c) {
                const float x = elem_f32<T, IsHalf>(at(tau, c));
                codes[tau * cw + c] = static_cast<uint8_t>(group_code(x, lo, s, vqmax));
            }
            if (half == 0) {
                const int64_t o = tok_row(L, b, h, dst_tok0 + tau) * vgroups + g;
                L.v_scale[o] = f32_to_f16(s);
                L.v_min[o] = f32_to_f16(lo);
            }
        }
    }
    __syncthreads();
    {
        const int words = L.v_words;
        const int per = 32 / vbits;
        int32_t* out = L.v_code + tok_row(L, b, h, dst_tok0) * words;
        for (int idx = threadIdx.x; idx < P * words; idx += kPackThreads) {
            const int tau = idx / words;
            const int w = idx % words;
            const uint8_t* crow = codes + tau * cw;
            uint32_t word = 0;
            for (int k = 0; k < per; ++k) {
                const int c = w * per + k;
                if (c < D) word |= static_cast<uint32_t>(crow[c]) << (k * vbits);
            }
            out[idx] = static_cast<int32_t>(word);
        }
    }
}

int pack_code_row(const lf_packed_layer& L);

// ---------------------------------------------------------------------------------------
// Fast path for the common shape: page = Key group = Value group = head_dim = 128, int2
// Values, 2-byte inputs with 16-byte aligned rows.  Two workgroups of 512 threads per page and
// kv head (blockIdx.z 0: Key page, 1: Value page -- every Key page is dispatched before the
// Value pages, ≈1 % faster than the reverse order at the current kernel; mixing the VALU-bound
// Key pages with the memory-bound Value pages measured slower, in alternate single blocks and in
// runs of 8), about 40 KB of LDS, of which the kernel's SGPR count lets three share a CU (56 KB
// and two for the widest tier mixes).  Per element the division uses a correctly rounded reciprocal of the group
// scale and one Markstein correction (div_rn); groups whose scale is not clamped above take the
// clamp-free magic_code.  The phases are listed at pack_fast_page.  Each integer tier has a
// 16-byte aligned segment of a token's code row (in slot order), so a word's 16 / 8 / 4 code
// bytes are one LDS read.
// ---------------------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kFastThreads = 512;
constexpr int kFastP = 128;
constexpr int kFastLd = 128;  // halves per staged row (unpadded: phase 1 reads one row per wave instruction)

// a / s rounded to nearest even from y = RN(1/s) (Markstein: q0 = RN(a*y) is within an ulp of
// a/s, the residual a - q0*s is exact by FMA, and RN(q0 + r*y) is the correctly rounded
// quotient when no step overflows or underflows).  ``a`` is clamped to FLT_MAX first: only a
// range that overflows float makes it +inf, and then s is clamped to 1e5, so the clamped
// quotient (>= 3.4e33) still clamps to qmax, as inf / s does; otherwise a <= s * qmax (s not
// clamped or clamped to 1e-5) or y = 1e-5, and a * y cannot overflow.  A quotient below the
// normal range rounds to code 0 either way.  (A CPU check of 40 M random, tie and overflow
// cases against IEEE division found no difference.)
__device__ __forceinline__ float div_rn(float a, float s, float y) {
    a = fminf(a, 3.40282347e38f);
    const float q0 = a * y;
    const float r = fmaf(-q0, s, a);
    return fmaf(r, y, q0);
}

// RN((hi - lo) / qmax) by div_rn on the constant inv = RN(1 / qmax), qmax one of 3, 15, 255: a
// range of +inf becomes FLT_MAX, whose quotient lies far above the clamp, as inf / qmax does.
// The group scale is clamp(raw, 1e-5, 1e5) (layout.py:16); in the subnormal range the clamp to
// 1e-5 hides the last bit.  (Checked on the CPU against IEEE division for 60 M ranges of every
// magnitude: no difference.)
__device__ __forceinline__ float raw_scale(float hi, float lo, float qmax, float inv) {
    return div_rn(hi - lo, qmax, inv);
}
__device__ __forceinline__ float clamp_scale(float raw) { return fminf(fmaxf(raw, 1e-5f), 1e5f); }

// code = clamp(rint((x - lo) / s), 0, qmax) with div_rn: the path for groups whose unclamped
// scale exceeds 1e5 (ranges above 1e5 qmax, infinite ones included).
__device__ __forceinline__ uint32_t fast_code(float x, float lo, float s, float y, float qmax) {
    const float q = __builtin_rintf(div_rn(x - lo, s, y));
    return static_cast<uint32_t>(__builtin_amdgcn_fmed3f(q, 0.0f, qmax));
}

// The common path, for groups whose unclamped scale r = RN(range / qmax) is at most 1e5: then
// s = max(r, 1e-5) >= range / qmax (1 - 2^-24), a = RN(x - lo) lies in [0, range], so a / s is
// at most qmax (1 + 2^-23) and its rint at most qmax -- the clamp cannot bind and nothing
// overflows.  The correctly rounded quotient plus 2^23 rounds to an integer, half to even, in
// the low mantissa bits: bits(q + 2^23) = 0x4B000000 + rint(q) for 0 <= q < 2^23, so the low
// byte is the code.  (A CPU check of 4 M groups of 32 values at every magnitude, ties and
// ranges around the 1e5 qmax boundary included, found no difference from the IEEE formula.)
__device__ __forceinline__ uint32_t magic_code(float x, float lo, float s, float y) {
    const float a = x - lo;
    const float q0 = a * y;
    const float r = fmaf(-q0, s, a);
    return __float_as_uint(fmaf(r, y, q0) + 8388608.0f);
}

// Sum over a 16-code word of the 0x4B000000 that each magic_code carries, shifted as its code
// is: a word built by adding magic codes shifted by 2 i, minus this, holds the codes.
constexpr uint32_t value_word_bias() {
    uint32_t s = 0;
    for (int i = 0; i < 16; ++i) s += 0x4B000000u << (2 * i);
    return s;
}

// min / max of three without the v_max_f32 x, x, x that the compiler puts before fminf / fmaxf
// of a value it cannot prove canonical (bf16 bits moved into a float's high half).  Quieting a
// signalling NaN is all that step does, and a NaN in a group is outside the packer's contract
// (the reference's own scale becomes NaN).
__device__ __forceinline__ float min3_raw(float a, float b, float c) {
    float d;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
    float d;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}

// The value of lane l ^ 1 / l ^ 2 (DPP quad_perm [1,0,3,2] / [2,3,0,1]).
__device__ __forceinline__ float quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));
}

// The two 16-bit elements of a dword as floats (element 0 in the low half).
template <bool IsHalf>
__device__ __forceinline__ void pair_f32(uint32_t d, float& e0, float& e1) {
    if constexpr (IsHalf) {
        e0 = f16_to_f32(static_cast<uint16_t>(d & 0xffffu));
        e1 = f16_to_f32(static_cast<uint16_t>(d >> 16));
    } else {
        e0 = __uint_as_float(d << 16);
        e1 = __uint_as_float(d & 0xffff0000u);
    }
}

// lo / hi of 32 values by 16 min3 / max3 each.
__device__ __forceinline__ void minmax32(const float (&v)[32], float& lo, float& hi) {
    lo = min3_raw(v[0], v[1], v[2]);
    hi = max3_raw(v[0], v[1], v[2]);
#pragma unroll
    for (int i = 3; i < 31; i += 2) {
        lo = min3_raw(lo, v[i], v[i + 1]);
        hi = max3_raw(hi, v[i], v[i + 1]);
    }
    lo = min3_raw(lo, v[31], v[31]);
    hi = max3_raw(hi, v[31], v[31]);
}

// Byte-per-code LDS row of the fast path: tier t's slots start at seg[t] (16-byte aligned).
struct CodeSegs {
    int seg[4];  // seg[3] = row bytes
};

__device__ __host__ inline CodeSegs code_segs(const lf_packed_layer& L) {
    CodeSegs s;
    s.seg[0] = 0;
    s.seg[1] = (L.k_width[0] + 15) & ~15;
    s.seg[2] = s.seg[1] + ((L.k_width[1] + 15) & ~15);
    s.seg[3] = s.seg[2] + ((L.k_width[2] + 15) & ~15);
    return s;
}

// The word helpers take code bytes in slot order whose bytes below the tier's count are codes
// (0..qmax) and whose later bytes may be stale page bytes: a stale byte only reaches bits of its
// own and later slots, which tier_words masks, so no byte needs masking before packing.

// 16 int2 codes (one per byte) -> LSB-first word: v_dot4_u32_u8 with weights 1, 4, 16, 64 puts
// a dword's four codes into its low byte (a code byte below 4 carries nothing into the next
// field; products of stale bytes only reach higher bits), and two byte permutes gather the four
// low bytes.
__device__ __forceinline__ uint32_t word_int2(uint4 b) {
    constexpr uint32_t kW = 0x40100401u;
    const uint32_t t0 = __builtin_amdgcn_udot4(b.x, kW, 0u, false), t1 = __builtin_amdgcn_udot4(b.y, kW, 0u, false);
    const uint32_t t2 = __builtin_amdgcn_udot4(b.z, kW, 0u, false), t3 = __builtin_amdgcn_udot4(b.w, kW, 0u, false);
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, 0x0c0c0400u);  // t0.byte0, t1.byte0, 0, 0
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, 0x04000c0cu);  // 0, 0, t2.byte0, t3.byte0
    return lo | hi;
}

// 8 int4 codes (one per byte) -> LSB-first word: x | x >> 4 puts codes 2k, 2k + 1 into byte 2k
// (a code byte below 16 carries nothing into the next field), one permute gathers bytes 0 and 2.
__device__ __forceinline__ uint32_t word_int4(uint2 b) {
    const uint32_t t0 = b.x | (b.x >> 4), t1 = b.y | (b.y >> 4);
    return __builtin_amdgcn_perm(t1, t0, 0x06040200u);
}

// Value page (layout.py:115-129): one quad per token row, lane w holding channels 32 w .. 32 w +
// 31 of token tid / 4; the row's min / max by two quad exchanges; lane w writes code words 2 w
// and 2 w + 1.  The page's 128 fp16 scales and mins are contiguous: gathered in LDS, each array
// leaves as one 256-byte store (token pairs; the row offset is even and the arrays 4-byte
// aligned, which the launcher checks).
template <bool IsHalf>
__device__ __forceinline__ void pack_value_page(const lf_packed_layer& L, const uint16_t* src, int64_t st, int b,
                                                int h, int64_t dst_tok0, unsigned char* smem) {
    const int tid = threadIdx.x;
    const int tk = tid >> 2, w = tid & 3;
    uint4 r[4];
    {
        const uint4* a = reinterpret_cast<const uint4*>(src + tk * st + 32 * w);
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = a[i];
    }
    float v[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pair_f32<IsHalf>(r[i].x, v[8 * i + 0], v[8 * i + 1]);
        pair_f32<IsHalf>(r[i].y, v[8 * i + 2], v[8 * i + 3]);
        pair_f32<IsHalf>(r[i].z, v[8 * i + 4], v[8 * i + 5]);
        pair_f32<IsHalf>(r[i].w, v[8 * i + 6], v[8 * i + 7]);
    }
    float lo, hi;
    minmax32(v, lo, hi);
    lo = min3_raw(lo, quad_xor1(lo), lo);
    hi = max3_raw(hi, quad_xor1(hi), hi);
    lo = min3_raw(lo, quad_xor2(lo), lo);
    hi = max3_raw(hi, quad_xor2(hi), hi);
    const float raw = raw_scale(hi, lo, 3.0f, 1.0f / 3.0f);
    const float sc = clamp_scale(raw);
    const float y = 1.0f / sc;
    uint32_t wd[2];
    if (raw <= 1e5f) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t acc = 0u - value_word_bias();
#pragma unroll
            for (int i = 0; i < 16; ++i) acc += magic_code(v[16 * j + i], lo, sc, y) << (2 * i);
            wd[j] = acc;
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t acc = 0;
#pragma unroll
            for (int i = 0; i < 16; ++i) acc |= fast_code(v[16 * j + i], lo, sc, y, 3.0f) << (2 * i);
            wd[j] = acc;
        }
    }
    reinterpret_cast<uint2*>(L.v_code + tok_row(L, b, h, dst_tok0 + tk) * 8)[w] = make_uint2(wd[0], wd[1]);
    uint16_t* vsm = reinterpret_cast<uint16_t*>(smem);  // [2][128]: scale, min
    if (w == 0) {
        vsm[tk] = f32_to_f16(sc);
        vsm[128 + tk] = f32_to_f16(lo);
    }
    __syncthreads();
    if (tid < 128) {
        uint16_t* dst = (tid < 64 ? L.v_scale : L.v_min) + tok_row(L, b, h, dst_tok0);
        reinterpret_cast<uint32_t*>(dst)[tid & 63] = reinterpret_cast<const uint32_t*>(vsm)[tid];
    }
}

// Code rows of the Key workgroup: one row of ``Ld`` bytes per token, Ld a compile-time constant
// so that phase 3's 32 byte stores per thread address by immediate offsets.  272 (17 x 16 bytes:
// consecutive rows start 4 banks apart) holds every tier mix whose int tiers' 16-byte aligned
// segments fit (all of the bench's), 400 the widest possible (3 x 128).
constexpr int kCodeLdNarrow = 272;
constexpr int kCodeLdWide = 400;
static_assert(kFastLd * 2 <= kCodeLdNarrow, "the staged page lies within the code rows");

__device__ __host__ inline int code_ld(const lf_packed_layer& L) {
    return code_segs(L).seg[3] <= kCodeLdNarrow ? kCodeLdNarrow : kCodeLdWide;
}

// LDS layout of the Key workgroup: the code rows (the staged page, 128 rows of 256 bytes,
// lies in their first 32 KB until phase 1 has read it), partial min/max, the channel map, the
// fp16 tier's channels, the page's block of the page-major Key scale/min copy (gathered here and
// stored as whole 16-byte chunks: at most 48 blocks of 32 bytes).
struct FastLds {
    int pmm, cpos, tidx, sm, total;
};

constexpr int kSmBlockMax = 48;  // 8-slot blocks of three integer tiers of at most 4 K-steps each

__device__ __host__ inline FastLds fast_lds(int ld, int w16) {
    FastLds f;
    f.pmm = kFastP * ld;                                 // after [128][ld] code bytes (ld % 16 == 0)
    f.cpos = f.pmm + 4 * 128 * 8;                        // [4][128] float2 -> [128] int16
    f.tidx = f.cpos + 128 * 2;                           // [w16] int16
    f.sm = f.tidx + ((w16 * 2 + 15) & ~15);              // [48][16] fp16 (16-byte aligned)
    f.total = f.sm + kSmBlockMax * 32 + 16;
    return f;
}

// Words of one integer tier (Bits 2, 4 or 8) of the Key page (layout.py:21-35, :94-97): with
// T = 512 / kw rows per pass, thread tid < T kw takes word w = tid % kw of rows tid / kw, + T,
// ...; word r kw + w of the page block is then tid, + T kw, ..., so consecutive threads store
// consecutive dwords and every store instruction covers whole lines.  Each word comes from
// 16 / 8 / 4 code bytes of its token's row; slots at or beyond the tier's count for this head
// are masked to 0 (layout.py:84-85).  tid / kw = (int)((tid + 0.5) * rcp(kw)): the hardware
// reciprocal's relative error (1 ulp) and the product's rounding leave the value within
// 512 / kw * 2^-21 of (tid + 0.5) / kw, which lies at least 1 / (2 kw) from an integer, so the
// truncation is exact for tid < 512.
template <int Bits, int Ld>
__device__ __forceinline__ void tier_words(const uint8_t* codes, int seg, int kw, int cnt, int32_t* out, int tid) {
    if (kw == 0) return;
    constexpr int kPer = 32 / Bits;
    const int T = kFastThreads / kw;
    if (tid >= T * kw) return;
    const int r0 = static_cast<int>((static_cast<float>(tid) + 0.5f) * __builtin_amdgcn_rcpf(static_cast<float>(kw)));
    const int w = tid - r0 * kw;
    const int nv = min(max(cnt - kPer * w, 0), kPer);
    const uint32_t keep = nv >= kPer ? 0xffffffffu : (1u << (Bits * nv)) - 1u;
    const uint8_t* src = codes + r0 * Ld + seg + kPer * w;
    int32_t* dst = out + tid;
    for (int r = r0; r < kFastP; r += T) {
        uint32_t word;
        if constexpr (Bits == 2) {
            word = word_int2(*reinterpret_cast<const uint4*>(src));
        } else if constexpr (Bits == 4) {
            word = word_int4(*reinterpret_cast<const uint2*>(src));
        } else {
            word = *reinterpret_cast<const uint32_t*>(src);
        }
        *dst = static_cast<int32_t>(word & keep);
        src += T * Ld;
        dst += T * kw;
    }
}

// One page of one kv head (blockIdx.y) of layer ``L``: the Key page or (``value``) the Value
// page.  Source rows tok0 .. tok0 + 127 of sequence b (element strides sb, sh, st) are
// written as page ``page`` of sequence b.  512 threads: four workgroups share a CU.
//   Value page  quad per token row (tid / 4), 32 channels per lane, read from global memory
//               directly (LDS only gathers the page's scales and mins)
//   Key page    stage (page -> LDS by LDS-DMA, tier tables -> channel map); phase 1: thread (channel
//               tid % 128, tokens 32 (tid / 128) + 0..31) min/max, the fp16 tier copied from
//               the staged page; phases 2, 3: the channel's scale and its 32 codes into byte
//               rows over the page; phase 4: the tiers' words (tier_words)
template <bool IsHalf, int Ld>
__device__ __forceinline__ void pack_fast_page(const lf_packed_layer& Lsrc, const void* k_src, const void* v_src,
                                               int64_t sb, int64_t sh, int64_t st, int b, int64_t tok0, int page,
                                               bool value) {
    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    // The layer descriptor and this head's tier counts, read before any store: the multi-layer
    // kernel's descriptor lives in device memory, which the page's stores might alias as far as
    // the compiler knows, so a field read after a store would be a vector load of its own round
    // trip (and the tier tables' pointers per lane a second one).
    const lf_packed_layer L = Lsrc;
    int tcnt[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) tcnt[t] = value || L.k_width[t] == 0 ? 0 : L.tier_count[t][h];
    // the page's block of the page-major scale/min copy (none: 0 blocks) and the tiers' first
    // blocks, in scalar registers before any store
    const bool has_sm = !value && L.k_sm_page != nullptr;
    const SmPage sp = sm_page(L.k_words);
    int sm_nb = has_sm ? sp.nb : 0, sm_b1 = sp.blk0[1], sm_b2 = sp.blk0[2];
    uint16_t* smg = has_sm ? L.k_sm_page + sm_page_idx(L, b, h, page) : nullptr;
    asm volatile("" : "+s"(sm_nb), "+s"(sm_b1), "+s"(sm_b2), "+s"(smg));
    const int64_t dst_tok0 = static_cast<int64_t>(page) * kFastP;
    constexpr int D = 128;
    extern __shared__ __align__(16) unsigned char smem[];

    if (value) {
        pack_value_page<IsHalf>(L, static_cast<const uint16_t*>(v_src) + b * sb + h * sh + tok0 * st, st, b, h,
                                dst_tok0, smem);
        return;
    }

    const FastLds fl = fast_lds(Ld, L.k_width[3]);
    uint8_t* codes = smem;                                                  // [128][Ld] code bytes
    uint16_t* kpage = reinterpret_cast<uint16_t*>(smem);                  // [128][128]: the page, read
                                                                            // before the codes replace it
    float2* pmm = reinterpret_cast<float2*>(smem + fl.pmm);                // [4][128] partial (lo, hi)
    int16_t* cpos = reinterpret_cast<int16_t*>(smem + fl.cpos);            // [128] code byte of a channel,
                                                                            // -1 - rank for the fp16 tier
    int16_t* tidx = reinterpret_cast<int16_t*>(smem + fl.tidx);            // [w16] channel of an fp16 slot
    uint16_t* smblk = reinterpret_cast<uint16_t*>(smem + fl.sm);           // the page's k_sm_page block
    const CodeSegs cs = code_segs(L);  // cs.seg[3] <= Ld (the launcher's choice of Ld)

    const int w0 = L.k_width[0], w1 = L.k_width[1], w2 = L.k_width[2], w16 = L.k_width[3];
    const int koff1 = w0, koff2 = w0 + w1, nslots = w0 + w1 + w2, wall = nslots + w16;
    // ---- stage the page and this head's tier tables (layout.py:49-68): all their global loads
    // go out before the first wait ----
    {
        // The page by LDS-DMA (buffer_load_dwordx4 ... lds): wave w's instruction i moves 1 KB
        // block k = 4 w + i, rows 4 k .. 4 k + 3, lane l's 16 bytes landing at 1024 k + 16 l.  The
        // row offset is the scalar soffset (rows are st apart in the source), the lane's part a
        // VGPR shared by the four instructions; the buffer word 3 0x00020000 (DATA_FORMAT 32)
        // is the gfx9 value for untyped accesses.  Offsets stay below 2^31 (st <= 2^22, checked
        // by the launcher).
        {
            const uint16_t* src = static_cast<const uint16_t*>(k_src) + b * sb + h * sh + tok0 * st;
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(src), 0, 0x7fffffff, 0x00020000);
            const int st2 = static_cast<int>(st) * 2;
            const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
            const int voff = (lane >> 4) * st2 + 16 * (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = 4 * wave + i;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(smem + 1024 * k), 16, voff, 4 * k * st2, 0, 0);
            }
        }
        // slot tid of tier t: its channel and the tier's count for head h (wall <= 512).
        // Constant indices into the layer descriptor only (a lane-dependent one would copy it to
        // scratch memory).
        int my_idx = 0, my_cnt = 0;
        if (tid < koff1) { my_idx = L.tier_index[0][h * w0 + tid]; my_cnt = tcnt[0]; }
        else if (tid < koff2) { my_idx = L.tier_index[1][h * w1 + tid - koff1]; my_cnt = tcnt[1]; }
        else if (tid < nslots) { my_idx = L.tier_index[2][h * w2 + tid - koff2]; my_cnt = tcnt[2]; }
        else if (tid < wall) { my_idx = L.tier_index[3][h * w16 + tid - nslots]; my_cnt = tcnt[3]; }
        // channel map: every channel sits in exactly one tier (rank < count), so every entry is
        // written once; padding slots (rank >= count): scale 1.0, min 0.0, code 0 (layout.py:84-85)
        if (tid < wall) {
            const int t = tid >= nslots ? 3 : tid >= koff2 ? 2 : tid >= koff1 ? 1 : 0;
            const int j = tid - (t == 3 ? nslots : t == 2 ? koff2 : t == 1 ? koff1 : 0);
            if (j < my_cnt) {
                cpos[my_idx] = static_cast<int16_t>(t == 3 ? -1 - j : (t == 2 ? cs.seg[2] : t == 1 ? cs.seg[1] : 0) + j);
                if (t == 3) tidx[j] = static_cast<int16_t>(my_idx);
            } else if (t < 3) {
                const int width = t == 2 ? w2 : t == 1 ? w1 : w0;
                const int64_t o = kgrp_idx(L, b, h, width, j, page);
                uint16_t* ks = t == 2 ? L.k_scale[2] : t == 1 ? L.k_scale[1] : L.k_scale[0];
                uint16_t* km = t == 2 ? L.k_min[2] : t == 1 ? L.k_min[1] : L.k_min[0];
                ks[o] = 0x3C00u;
                km[o] = 0;
            }
        }
        // page-major copy (k_sm_page), gathered in LDS: positions of no channel of this head --
        // ranks at or past the tier's count, padding ranks of a block -- hold scale 1.0, min 0.0;
        // the channels' own positions are written with their scales in phase 2
        if (tid < 8 * sm_nb) {
            const int gb = tid >> 3, pos = tid & 7;
            const int t = gb >= sm_b2 ? 2 : gb >= sm_b1 ? 1 : 0;
            const int j = sm_slot(t, gb - (t == 2 ? sm_b2 : t == 1 ? sm_b1 : 0), pos);
            if (j >= tcnt[t]) {
                smblk[16 * gb + pos] = 0x3C00u;
                smblk[16 * gb + 8 + pos] = 0;
            }
        }
        __syncthreads();
    }

    // ---- phase 1: Key min/max of channel c over tokens 32 ck .. 32 ck + 31 ----
    const int c = tid & (D - 1), ck = tid >> 7;
    const int pos = cpos[c];
    float x[32];
    {
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = elem_f32<uint16_t, IsHalf>(kpage[(32 * ck + i) * kFastLd + c]);
        float lo, hi;
        minmax32(x, lo, hi);
        pmm[ck * D + c] = float2{lo, hi};
    }
    // fp16 tier (layout.py:101-111; exact for fp16 input, RNE for bf16) straight from the staged
    // page, element i = (token i / w16, slot i % w16) in memory order; padding slots are 0
    if (w16 > 0) {
        const int cnt = tcnt[3];
        // i / w16 as in tier_words: within 2^14 / w16 * 2^-21 of (i + 0.5) / w16, at least
        // 1 / (2 w16) from an integer, for i < 128 w16
        const float rk = __builtin_amdgcn_rcpf(static_cast<float>(w16));
        uint16_t* out = L.k_value16 + tok_row(L, b, h, dst_tok0) * w16;
        for (int i = tid; i < kFastP * w16; i += kFastThreads) {
            const int tau = static_cast<int>((static_cast<float>(i) + 0.5f) * rk), j = i - tau * w16;
            out[i] = j < cnt ? f32_to_f16(elem_f32<uint16_t, IsHalf>(kpage[tau * kFastLd + tidx[j]]))
                             : static_cast<uint16_t>(0);
        }
    }
    __syncthreads();  // the page is dead: the code rows may overwrite it

    // ---- phases 2, 3: the channel's group scale (layout.py:12-18) and its 32 codes; bytes of
    // slots no channel writes are masked when the words are assembled ----
    if (pos >= 0) {
        const float2 m0 = pmm[c], m1 = pmm[D + c], m2 = pmm[2 * D + c], m3 = pmm[3 * D + c];
        const float lo = min3_raw(min3_raw(m0.x, m1.x, m2.x), m3.x, m3.x);
        const float hi = max3_raw(max3_raw(m0.y, m1.y, m2.y), m3.y, m3.y);
        const int t = pos >= cs.seg[2] ? 2 : pos >= cs.seg[1] ? 1 : 0;
        const float qmax = t == 2 ? 255.0f : t == 1 ? 15.0f : 3.0f;
        const float raw = raw_scale(hi, lo, qmax, t == 2 ? 1.0f / 255.0f : t == 1 ? 1.0f / 15.0f : 1.0f / 3.0f);
        const float sc = clamp_scale(raw);
        const float y = 1.0f / sc;
        if (ck == 0) {
            const int j = pos - (t == 2 ? cs.seg[2] : t == 1 ? cs.seg[1] : 0);
            const int width = t == 2 ? w2 : t == 1 ? w1 : w0;
            const int64_t o = kgrp_idx(L, b, h, width, j, page);
            uint16_t* ks = t == 2 ? L.k_scale[2] : t == 1 ? L.k_scale[1] : L.k_scale[0];
            uint16_t* km = t == 2 ? L.k_min[2] : t == 1 ? L.k_min[1] : L.k_min[0];
            const uint16_t hs = f32_to_f16(sc), hl = f32_to_f16(lo);
            ks[o] = hs;
            km[o] = hl;
            if (sm_nb != 0) {
                int lb, bp;
                sm_place(t, j, lb, bp);
                uint16_t* blk = smblk + 16 * ((t == 2 ? sm_b2 : t == 1 ? sm_b1 : 0) + lb);
                blk[bp] = hs;
                blk[8 + bp] = hl;
            }
        }
        uint8_t* crow = codes + (32 * ck) * Ld + pos;
        if (raw <= 1e5f) {
#pragma unroll
            for (int i = 0; i < 32; ++i) crow[i * Ld] = static_cast<uint8_t>(magic_code(x[i], lo, sc, y));
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) crow[i * Ld] = static_cast<uint8_t>(fast_code(x[i], lo, sc, y, qmax));
        }
    }
    __syncthreads();

    // ---- phase 4: the integer tiers' words; the page-major scale/min block leaves as 16-byte chunks ----
    if (tid < 2 * sm_nb) reinterpret_cast<uint4*>(smg)[tid] = reinterpret_cast<const uint4*>(smblk)[tid];
    const int64_t row0 = tok_row(L, b, h, dst_tok0);
    const int kw0 = L.k_words[0], kw1 = L.k_words[1], kw2 = L.k_words[2];
    tier_words<2, Ld>(codes, 0, kw0, tcnt[0], L.k_code[0] + row0 * kw0, tid);
    tier_words<4, Ld>(codes, cs.seg[1], kw1, tcnt[1], L.k_code[1] + row0 * kw1, tid);
    tier_words<8, Ld>(codes, cs.seg[2], kw2, tcnt[2], L.k_code[2] + row0 * kw2, tid);
}

template <bool IsHalf, int Ld>
__global__ __launch_bounds__(kFastThreads) void pack_fast_kernel(PackJobArgs a) {
    const int job = blockIdx.x;
    pack_fast_page<IsHalf, Ld>(a.L, a.k_src, a.v_src, a.sb, a.sh, a.st, a.jobs[3 * job + 0], a.jobs[3 * job + 1],
                           a.jobs[3 * job + 2], blockIdx.z == 1);
}

// Several layers' pages in one launch: job = (layer, b, src_token0, dst_page); the layer's
// descriptor and page source are read from device memory.
struct PackMultiArgs {
    const lf_packed_layer* layers;
    const lf_pack_source* srcs;
    const int32_t* jobs;
};

template <bool IsHalf, int Ld>
__global__ __launch_bounds__(kFastThreads) void pack_fast_multi_kernel(PackMultiArgs m) {
    const int job = blockIdx.x;
    const int layer = __builtin_amdgcn_readfirstlane(m.jobs[4 * job + 0]);
    const lf_packed_layer& L = m.layers[layer];
    const lf_pack_source& S = m.srcs[layer];
    pack_fast_page<IsHalf, Ld>(L, S.k, S.v, S.stride_b, S.stride_h, S.stride_t, m.jobs[4 * job + 1], m.jobs[4 * job + 2],
                           m.jobs[4 * job + 3], blockIdx.z == 1);
}

// ``st``: the source's token stride in elements (the Key page is read through a buffer resource
// whose byte offsets, up to 127 st 2 + 256, must stay below 2^31).
bool pack_fast_ok(const lf_packed_layer& L, int src_dtype, bool vec16, int64_t st) {
    return vec16 && src_dtype != LF_FP32 && st > 0 && st <= (1 << 22) && L.head_dim == 128 && L.page_size == kFastP && L.k_group == kFastP &&
           L.v_group == 128 && L.bit_v == 2 && L.v_groups == 1 && L.v_words == 8 && L.cap_tokens % 2 == 0 &&
           (reinterpret_cast<uintptr_t>(L.v_scale) & 3) == 0 && (reinterpret_cast<uintptr_t>(L.v_min) & 3) == 0 &&
           (reinterpret_cast<uintptr_t>(L.v_code) & 7) == 0;
}

size_t pack_fast_lds_bytes(int ld, int w16) { return static_cast<size_t>(fast_lds(ld, w16).total); }

// One fast-path launch of kernel ``K`` (pack_fast_kernel or pack_fast_multi_kernel instances for
// bf16 / fp16 sources) with ``lds`` bytes of dynamic LDS.
template <typename Args>
int launch_fast(const void* fn_bf16, const void* fn_f16, void (*k_bf16)(Args), void (*k_f16)(Args), bool half,
                dim3 grid, size_t lds, const Args& args, hipStream_t stream) {
    const int rc = allow_dynamic_lds(half ? fn_f16 : fn_bf16, lds);
    if (rc != LF_OK) return rc;
    if (half) hipLaunchKernelGGL(k_f16, grid, dim3(kFastThreads), lds, stream, args);
    else hipLaunchKernelGGL(k_bf16, grid, dim3(kFastThreads), lds, stream, args);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

template <int Ld>
int launch_fast_single(const PackJobArgs& a, bool half, dim3 grid, size_t lds, hipStream_t stream) {
    return launch_fast<PackJobArgs>(reinterpret_cast<const void*>(&pack_fast_kernel<false, Ld>),
                                    reinterpret_cast<const void*>(&pack_fast_kernel<true, Ld>),
                                    pack_fast_kernel<false, Ld>, pack_fast_kernel<true, Ld>, half, grid, lds, a,
                                    stream);
}

template <int Ld>
int launch_fast_multi(const PackMultiArgs& m, bool half, dim3 grid, size_t lds, hipStream_t stream) {
    return launch_fast<PackMultiArgs>(reinterpret_cast<const void*>(&pack_fast_multi_kernel<false, Ld>),
                                      reinterpret_cast<const void*>(&pack_fast_multi_kernel<true, Ld>),
                                      pack_fast_multi_kernel<false, Ld>, pack_fast_multi_kernel<true, Ld>, half, grid,
                                      lds, m, stream);
}

int pack_code_row(const lf_packed_layer& L) {
    const int wsum = L.k_width[0] + L.k_width[1] + L.k_width[2];
    return wsum > L.head_dim ? wsum : L.head_dim;
}

// Dynamic LDS of the generic kernel: the staged page (when ``staged``), the code rows and the
// per-channel tier maps.
size_t pack_lds_bytes(const lf_packed_layer& L, int elem, bool staged) {
    const int D = L.head_dim;
    const int ld = D + (elem == 2 ? 2 : 1);
    return (staged ? static_cast<size_t>(L.page_size) * ld * elem : 0) +
           static_cast<size_t>(L.page_size) * pack_code_row(L) + ((D + 1) & ~1) + 2 * D + 16;
}

template <typename T, bool IsHalf>
int launch_one(const PackJobArgs& a, dim3 grid, int elem, hipStream_t stream) {
    const bool staged = pack_lds_bytes(a.L, elem, true) <= 160 * 1024;
    const size_t lds = pack_lds_bytes(a.L, elem, staged);
    if (lds > 160 * 1024) return LF_E_SHAPE;
    const void* fn = staged ? reinterpret_cast<const void*>(&pack_pages_kernel<T, IsHalf, true>)
                            : reinterpret_cast<const void*>(&pack_pages_kernel<T, IsHalf, false>);
    const int rc = allow_dynamic_lds(fn, lds);
    if (rc != LF_OK) return rc;
    if (staged) hipLaunchKernelGGL((pack_pages_kernel<T, IsHalf, true>), grid, dim3(kPackThreads), lds, stream, a);
    else hipLaunchKernelGGL((pack_pages_kernel<T, IsHalf, false>), grid, dim3(kPackThreads), lds, stream, a);
    return LF_OK;
}

}  // namespace

int launch_pack_pages(const lf_packed_layer& L, const void* k_src, const void* v_src, int src_dtype,
                      int64_t sb, int64_t sh, int64_t st, const int32_t* jobs, int n_jobs,
                      hipStream_t stream) {
    PackJobArgs a;
    a.L = L;
    a.k_src = k_src;
    a.v_src = v_src;
    a.sb = sb;
    a.sh = sh;
    a.st = st;
    a.jobs = jobs;
    const int elem = src_dtype == LF_FP32 ? 4 : 2;
    const uintptr_t kp = reinterpret_cast<uintptr_t>(k_src), vp = reinterpret_cast<uintptr_t>(v_src);
    a.vec16 = ((kp | vp) % 16 == 0) && ((sb * elem) % 16 == 0) && ((sh * elem) % 16 == 0) &&
              ((st * elem) % 16 == 0);
    a.cw = pack_code_row(L);
    dim3 grid(n_jobs, L.n_kv);
    if (pack_fast_ok(L, src_dtype, a.vec16 != 0, st)) {
        const int ld = code_ld(L);
        const size_t lds = pack_fast_lds_bytes(ld, L.k_width[3]);
        const bool half = src_dtype == LF_FP16;
        const dim3 grid2(n_jobs, L.n_kv, 2);  // z: Key page, Value page
        return ld == kCodeLdNarrow ? launch_fast_single<kCodeLdNarrow>(a, half, grid2, lds, stream)
                                   : launch_fast_single<kCodeLdWide>(a, half, grid2, lds, stream);
    }
    int rc;
    if (src_dtype == LF_BF16) rc = launch_one<uint16_t, false>(a, grid, elem, stream);
    else if (src_dtype == LF_FP16) rc = launch_one<uint16_t, true>(a, grid, elem, stream);
    else if (src_dtype == LF_FP32) rc = launch_one<float, false>(a, grid, elem, stream);
    else return LF_E_DTYPE;
    if (rc != LF_OK) return rc;
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

int launch_pack_pages_multi(const lf_packed_layer* layers_dev, const lf_packed_layer* layers_host,
                            const lf_pack_source* srcs_dev, const lf_pack_source* srcs_host, int n_layers,
                            int src_dtype, const int32_t* jobs, int n_jobs, hipStream_t stream) {
    if (src_dtype == LF_FP32) return LF_E_UNSUPPORTED;
    int ld = kCodeLdNarrow;
    for (int i = 0; i < n_layers; ++i) {
        const lf_packed_layer& L = layers_host[i];
        const lf_pack_source& S = srcs_host[i];
        if (L.n_kv != layers_host[0].n_kv) return LF_E_UNSUPPORTED;  // one grid shape for all layers
        const uintptr_t kp = reinterpret_cast<uintptr_t>(S.k), vp = reinterpret_cast<uintptr_t>(S.v);
        const bool vec16 = ((kp | vp) % 16 == 0) && ((S.stride_b * 2) % 16 == 0) && ((S.stride_h * 2) % 16 == 0) &&
                           ((S.stride_t * 2) % 16 == 0);
        if (!pack_fast_ok(L, src_dtype, vec16, S.stride_t)) return LF_E_UNSUPPORTED;
        if (code_ld(L) == kCodeLdWide) ld = kCodeLdWide;
    }
    size_t lds = 0;
    for (int i = 0; i < n_layers; ++i) {
        const size_t l = pack_fast_lds_bytes(ld, layers_host[i].k_width[3]);
        lds = l > lds ? l : lds;
    }
    const bool half = src_dtype == LF_FP16;
    PackMultiArgs m{layers_dev, srcs_dev, jobs};
    const dim3 grid(n_jobs, layers_host[0].n_kv, 2);  // z: Key page, Value page
    return ld == kCodeLdNarrow ? launch_fast_multi<kCodeLdNarrow>(m, half, grid, lds, stream)
                               : launch_fast_multi<kCodeLdWide>(m, half, grid, lds, stream);
}

}  // namespace lf
