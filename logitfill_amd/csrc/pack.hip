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

template <typename T, bool IsHalf>
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
    uint8_t* codes = smem + static_cast<size_t>(P) * ld * sizeof(T);     // [P][cw]
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
    stage_page<T>(page_lds, ld, ksrc, a.st, P, D, a.vec16 != 0);
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
                const float x = elem_f32<T, IsHalf>(page_lds[tau * ld + c]);
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
                const float x = elem_f32<T, IsHalf>(page_lds[tau * ld + c]);
                crow[tau * cw] = static_cast<uint8_t>(group_code(x, lo, s, qmax));
            }
            if (half == 0) {
                const int64_t o = kgrp_idx(L, b, h, L.k_width[t], j, grp0 + g);
                L.k_scale[t][o] = f32_to_f16(s);
                L.k_min[t][o] = f32_to_f16(lo);
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
                if constexpr (IsHalf) v = static_cast<uint16_t>(page_lds[tau * ld + c]);
                else v = f32_to_f16(elem_f32<T, IsHalf>(page_lds[tau * ld + c]));
            }
            out[idx] = v;
        }
    }
    __syncthreads();

    // ---- Value page (layout.py:115-129) ----
    const T* vsrc = static_cast<const T*>(a.v_src) + b * a.sb + h * a.sh + tok0 * a.st;
    stage_page<T>(page_lds, ld, vsrc, a.st, P, D, a.vec16 != 0);
    __syncthreads();

    if (L.bit_v >= 16) {
        uint16_t* out = L.v_value16 + tok_row(L, b, h, dst_tok0) * D;
        for (int idx = threadIdx.x; idx < P * D; idx += kPackThreads) {
            const int tau = idx / D;
            const int c = idx % D;
            if constexpr (IsHalf) out[idx] = static_cast<uint16_t>(page_lds[tau * ld + c]);
            else out[idx] = f32_to_f16(elem_f32<T, IsHalf>(page_lds[tau * ld + c]));
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
                const float x = elem_f32<T, IsHalf>(page_lds[tau * ld + c]);
                lo = fminf(lo, x);
                hi = fmaxf(hi, x);
            }
        }
        lo = fminf(lo, __shfl_xor(lo, 1, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, 1, kWave));
        if (live) {
            const float s = group_scale(hi, lo, vqmax);
            for (int c = beg; c < end; ++c) {
                const float x = elem_f32<T, IsHalf>(page_lds[tau * ld + c]);
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

int pack_code_row(const lf_packed_layer& L) {
    const int wsum = L.k_width[0] + L.k_width[1] + L.k_width[2];
    return wsum > L.head_dim ? wsum : L.head_dim;
}

size_t pack_lds_bytes(const lf_packed_layer& L, int elem) {
    const int D = L.head_dim;
    const int ld = D + (elem == 2 ? 2 : 1);
    return static_cast<size_t>(L.page_size) * ld * elem +
           static_cast<size_t>(L.page_size) * pack_code_row(L) + ((D + 1) & ~1) + 2 * D + 16;
}

template <typename T, bool IsHalf>
int launch_one(const PackJobArgs& a, dim3 grid, size_t lds, hipStream_t stream) {
    static size_t lds_limit = 64 * 1024;
    if (lds > lds_limit) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&pack_pages_kernel<T, IsHalf>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (e != hipSuccess) return static_cast<int>(e);
        lds_limit = lds;
    }
    hipLaunchKernelGGL((pack_pages_kernel<T, IsHalf>), grid, dim3(kPackThreads), lds, stream, a);
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
    const size_t lds = pack_lds_bytes(L, elem);
    if (lds > 160 * 1024) return LF_E_SHAPE;
    dim3 grid(n_jobs, L.n_kv);
    int rc;
    if (src_dtype == LF_BF16) rc = launch_one<uint16_t, false>(a, grid, lds, stream);
    else if (src_dtype == LF_FP16) rc = launch_one<uint16_t, true>(a, grid, lds, stream);
    else if (src_dtype == LF_FP32) rc = launch_one<float, false>(a, grid, lds, stream);
    else return LF_E_DTYPE;
    if (rc != LF_OK) return rc;
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
