// Shared device helpers for the logitfill_amd HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/logitfill_amd.h"

namespace lf {

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

// ---- scalar conversions -------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t x) {
    _Float16 h;
    __builtin_memcpy(&h, &x, 2);
    return static_cast<float>(h);
}

// Round to nearest even, overflow to +-inf (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint16_t f32_to_f16(float x) {
    _Float16 h = static_cast<_Float16>(x);
    uint16_t r;
    __builtin_memcpy(&r, &h, 2);
    return r;
}

// Round to nearest even; NaN stays NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float x) {
    uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// Load element ``i`` of a tensor of lf_dtype ``dt`` as float.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
    if (dt == LF_BF16) return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    if (dt == LF_FP16) return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dt, float v) {
    if (dt == LF_BF16) static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    else if (dt == LF_FP16) static_cast<uint16_t*>(p)[i] = f32_to_f16(v);
    else static_cast<float*>(p)[i] = v;
}

// ---- launch helpers -------------------------------------------------------

// Allow ``bytes`` of dynamic LDS for kernel ``fn`` on the current device; launches above
// 64 KB need the attribute.  Called before every such launch (a host-side call on the
// function's per-device state), so the library itself caches nothing.
inline int allow_dynamic_lds(const void* fn, size_t bytes) {
    if (bytes <= 64 * 1024) return LF_OK;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    return e == hipSuccess ? LF_OK : static_cast<int>(e);
}

// ---- wave reductions ----------------------------------------------------

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// ---- layout offsets (reference byte layout, capacity strided) -----------

// Row (b, h, token) of a [batch][n_kv][cap_tokens][...] array.
__device__ __forceinline__ int64_t tok_row(const lf_packed_layer& L, int b, int h, int64_t tok) {
    return (static_cast<int64_t>(b) * L.n_kv + h) * L.cap_tokens + tok;
}

// Element (b, h, j, grp) of a [batch][n_kv][width][cap_kgroups] array.
__device__ __forceinline__ int64_t kgrp_idx(const lf_packed_layer& L, int b, int h, int width, int j,
                                            int64_t grp) {
    return ((static_cast<int64_t>(b) * L.n_kv + h) * width + j) * L.cap_kgroups + grp;
}

// ---- page-major Key scale/min copy (k_sm_page) ---------------------------------------------
//
// The matrix-core decode kernel reads a page's Key scales and mins as one contiguous block per
// (sequence, kv head, page): the integer tiers' slots in its K-step order, 8-slot blocks, each
// block's 8 fp16 scales then its 8 fp16 mins (32 bytes).  Tier t's blocks start at block
// sm_blk0[t]; K-steps of 4 blocks: int2 2 * ceil(words / 4) (a step takes half of 4 words), int4
// ceil(words / 4), int8 ceil(ceil(words / 2) / 4).  Positions whose slot is not a real channel of
// the head (rank >= count, or past the tier's words) hold scale 1.0, min 0.0.

struct SmPage {
    int blk0[3];  // first block of tier t
    int nb;       // blocks of the integer tiers
};

__host__ __device__ inline SmPage sm_page(const int32_t (&k_words)[3]) {
    SmPage s;
    const int kst0 = 2 * ((k_words[0] + 3) / 4), kst1 = (k_words[1] + 3) / 4, kst2 = ((k_words[2] + 1) / 2 + 3) / 4;
    s.blk0[0] = 0;
    s.blk0[1] = 4 * kst0;
    s.blk0[2] = 4 * (kst0 + kst1);
    s.nb = 4 * (kst0 + kst1 + kst2);
    return s;
}

// uint16 elements of one page's block: nb x (8 scales + 8 mins).
__host__ __device__ inline int sm_page_elems(const int32_t (&k_words)[3]) { return 16 * sm_page(k_words).nb; }

// Tier-local rank of position ``pos`` (0..7) of tier block ``lb``: the order in which the
// decode kernel's code unpack yields a block's 8 codes (int2: word 4 (lb / 8) + lb % 4, half
// (lb / 4) % 2, codes (4 half + r, 4 half + r + 8) for pos 2 r, 2 r + 1; int4: word lb, codes
// (r, r + 4); int8: words 2 lb, 2 lb + 1, bytes (r & 1, + 2)).
__host__ __device__ inline int sm_slot(int tier, int lb, int pos) {
    const int r = pos >> 1, odd = pos & 1;
    if (tier == 0) {
        const int word = 4 * (lb >> 3) + (lb & 3), half = (lb >> 2) & 1;
        return 16 * word + 4 * half + r + 8 * odd;
    }
    if (tier == 1) return 8 * lb + r + 4 * odd;
    if (tier == 2) return 4 * (2 * lb + (r >> 1)) + (r & 1) + 2 * odd;
    return 8 * lb + pos;  // fp16 tier: natural order
}

// Inverse of sm_slot for the integer tiers: the block (lb) and position of rank j.
__host__ __device__ inline void sm_place(int tier, int j, int& lb, int& pos) {
    if (tier == 0) {
        const int word = j >> 4, q = j & 15, odd = q >> 3, half = (q >> 2) & 1, r = q & 3;
        lb = 8 * (word >> 2) + 4 * half + (word & 3);
        pos = 2 * r + odd;
    } else if (tier == 1) {
        const int q = j & 7;
        lb = j >> 3;
        pos = 2 * (q & 3) + (q >> 2);
    } else {
        const int q = j & 7, r = 2 * (q >> 2) + (q & 1), odd = (q >> 1) & 1;
        lb = j >> 3;
        pos = 2 * r + odd;
    }
}

// First element of page ``page``'s block of (b, h) in k_sm_page [batch][n_kv][cap_kgroups][elems].
__host__ __device__ inline int64_t sm_page_idx(const lf_packed_layer& L, int b, int h, int64_t page) {
    return ((static_cast<int64_t>(b) * L.n_kv + h) * L.cap_kgroups + page) * sm_page_elems(L.k_words);
}

}  // namespace lf
