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

}  // namespace lf
