// Dense float32 reconstruction of one sequence's packed history.
//
// Reference: dequantize_key / dequantize_value, src/logitfill/packed/layout.py:132-182
// (restored = code * scale + min with float16 scale/min upcast; the fp16 tier
// upcast as stored).  The product of code and scale and the add of min are
// separately rounded, as in the reference's torch arithmetic.
#pragma clang fp contract(off)

#include "lf_common.hpp"

namespace lf {
namespace {

struct DequantArgs {
    lf_packed_layer L;
    int b;
    int tokens;
    float* k_out;
    float* v_out;
};

// One thread per (head, token, channel) element of K and of V.
__global__ __launch_bounds__(256) void dequant_kernel(DequantArgs a) {
    const lf_packed_layer& L = a.L;
    const int D = L.head_dim;
    const int h = blockIdx.y;
    const int64_t n = static_cast<int64_t>(a.tokens) * D;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int tok = static_cast<int>(e / D);
        const int c = static_cast<int>(e % D);
        const int64_t row = tok_row(L, a.b, h, tok);
        const int64_t oi = (static_cast<int64_t>(h) * a.tokens + tok) * D + c;
        // Key: find the channel's tier and rank (tables are tiny; linear scan).
        float kv = 0.f;
        for (int t = 0; a.k_out && t < 4; ++t) {
            const int w = L.k_width[t];
            if (w == 0) continue;
            const int cnt = L.tier_count[t][h];
            const int* idx = L.tier_index[t] + h * w;
            int j = -1;
            for (int q = 0; q < cnt; ++q)
                if (idx[q] == c) { j = q; break; }
            if (j < 0) continue;
            if (t == 3) {
                kv = f16_to_f32(L.k_value16[row * w + j]);
            } else {
                const int bits = 2 << t;
                const int per = 32 / bits;
                const uint32_t word = static_cast<uint32_t>(L.k_code[t][row * L.k_words[t] + j / per]);
                const float code = static_cast<float>((word >> ((j % per) * bits)) & ((1u << bits) - 1u));
                const int64_t gi = kgrp_idx(L, a.b, h, w, j, tok / L.k_group);
                const float prod = code * f16_to_f32(L.k_scale[t][gi]);
                kv = prod + f16_to_f32(L.k_min[t][gi]);
            }
            break;
        }
        if (a.k_out) a.k_out[oi] = kv;
        if (!a.v_out) continue;
        float vv;
        if (L.bit_v >= 16) {
            vv = f16_to_f32(L.v_value16[row * D + c]);
        } else {
            const int bits = L.bit_v;
            const int per = 32 / bits;
            const uint32_t word = static_cast<uint32_t>(L.v_code[row * L.v_words + c / per]);
            const float code = static_cast<float>((word >> ((c % per) * bits)) & ((1u << bits) - 1u));
            const int gi = c / L.v_group;
            const float prod = code * f16_to_f32(L.v_scale[row * L.v_groups + gi]);
            vv = prod + f16_to_f32(L.v_min[row * L.v_groups + gi]);
        }
        a.v_out[oi] = vv;
    }
}

}  // namespace

int launch_dequantize(const lf_packed_layer& L, int b, int tokens, float* k_out, float* v_out,
                      hipStream_t stream) {
    DequantArgs a{L, b, tokens, k_out, v_out};
    const int64_t n = static_cast<int64_t>(tokens) * L.head_dim;
    int blocks = static_cast<int>((n + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    hipLaunchKernelGGL(dequant_kernel, dim3(blocks, L.n_kv), dim3(256), 0, stream, a);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
