// Element-wise layout helpers of the packed format on the device:
//   asymmetric_codes  (reference src/logitfill/packed/layout.py:12-18)
//   pack_ints         (layout.py:21-35)
//   unpack_ints       (layout.py:38-46)
// They are the building blocks the page packers use; exposed on their own for callers of
// the reference's layout module.  Compiled without FP contraction: every subtraction and
// the division are separately rounded IEEE float32 operations, as in the reference's torch
// arithmetic on float32 tensors.
#pragma clang fp contract(off)

#include "lf_common.hpp"

namespace lf {
namespace {

// One wave per group: lanes stride over the group for min / max (a wave reduction), then
// every lane codes its elements.  s = clamp((hi - lo) / qmax, 1e-5, 1e5);
// code = clamp(rint_half_even((x - lo) / s), 0, qmax).
__global__ __launch_bounds__(256) void asym_codes_kernel(const void* x, int dtype, int64_t n_groups, int group,
                                                          int bits, int32_t* codes, float* scale, float* lo_out) {
    const int lane = threadIdx.x & 63;
    const int64_t grp = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (grp >= n_groups) return;
    const int64_t base = grp * group;
    float lo = __builtin_inff(), hi = -__builtin_inff();
    for (int i = lane; i < group; i += kWave) {
        const float v = load_as_f32(x, base + i, dtype);
        lo = fminf(lo, v);
        hi = fmaxf(hi, v);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        lo = fminf(lo, __shfl_xor(lo, off, kWave));
        hi = fmaxf(hi, __shfl_xor(hi, off, kWave));
    }
    const float qmax = static_cast<float>((1 << bits) - 1);
    const float s = fminf(fmaxf((hi - lo) / qmax, 1e-5f), 1e5f);
    for (int i = lane; i < group; i += kWave) {
        const float q = __builtin_rintf((load_as_f32(x, base + i, dtype) - lo) / s);
        codes[base + i] = static_cast<int32_t>(fminf(fmaxf(q, 0.f), qmax));
    }
    if (lane == 0) {
        scale[grp] = s;
        lo_out[grp] = lo;
    }
}

// One thread per output word: slot j of a row lands in word j / per at bit (j % per) * bits.
__global__ __launch_bounds__(256) void pack_ints_kernel(const int32_t* codes, int64_t rows, int n, int bits,
                                                         int n_words, int32_t* words) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= rows * n_words) return;
    const int64_t r = e / n_words;
    const int w = static_cast<int>(e - r * n_words);
    const int per = 32 / bits;
    uint32_t word = 0;
    for (int k = 0; k < per; ++k) {
        const int j = w * per + k;
        if (j < n) word |= static_cast<uint32_t>(codes[r * n + j]) << (k * bits);
    }
    words[e] = static_cast<int32_t>(word);
}

// One thread per output code.
__global__ __launch_bounds__(256) void unpack_ints_kernel(const int32_t* words, int64_t rows, int n_words, int count,
                                                           int bits, int32_t* codes) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (e >= rows * count) return;
    const int64_t r = e / count;
    const int j = static_cast<int>(e - r * count);
    const int per = 32 / bits;
    const uint32_t word = static_cast<uint32_t>(words[r * n_words + j / per]);
    const uint32_t mask = bits >= 32 ? 0xffffffffu : (1u << bits) - 1u;  // 1u << 32 is undefined
    codes[e] = static_cast<int32_t>((word >> ((j % per) * bits)) & mask);
}

int grid_for(int64_t n, int per_block) {
    const int64_t blocks = (n + per_block - 1) / per_block;
    return static_cast<int>(blocks);
}

}  // namespace

int launch_asymmetric_codes(const void* x, int dtype, int64_t n_groups, int group, int bits, int32_t* codes,
                            float* scale, float* lo, hipStream_t stream) {
    hipLaunchKernelGGL(asym_codes_kernel, dim3(grid_for(n_groups, 4)), dim3(256), 0, stream, x, dtype, n_groups, group,
                       bits, codes, scale, lo);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

int launch_pack_ints(const int32_t* codes, int64_t rows, int n, int bits, int32_t* words, hipStream_t stream) {
    const int per = 32 / bits;
    const int n_words = (n + per - 1) / per;
    hipLaunchKernelGGL(pack_ints_kernel, dim3(grid_for(rows * n_words, 256)), dim3(256), 0, stream, codes, rows, n, bits,
                       n_words, words);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

int launch_unpack_ints(const int32_t* words, int64_t rows, int n_words, int count, int bits, int32_t* codes,
                       hipStream_t stream) {
    hipLaunchKernelGGL(unpack_ints_kernel, dim3(grid_for(rows * count, 256)), dim3(256), 0, stream, words, rows, n_words,
                       count, bits, codes);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
