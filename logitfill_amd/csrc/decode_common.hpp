// Split-K decode: work items, partial results and the fused cross-split merge.
//
// A decode launch covers work items (b, page_begin, page_end, kind) x kv heads.
// Each workgroup produces, for the g = n_q / n_kv query heads of its kv head,
// a partial (m, l, o[D]) over its tokens: m the running max of the log2-domain
// scores, l = sum 2^(s - m), o = sum 2^(s - m) v.  The last workgroup of a
// (sequence, kv head) to finish -- counted with a device-scope atomic -- merges
// the partials (flash-decoding reduce) and writes the output; it then resets
// the counter so the workspace needs no clearing between calls.
#pragma once

#include "lf_common.hpp"

namespace lf {

struct DecodeParams {
    lf_packed_layer L;
    lf_decode_args A;
    int g;          // query heads per kv head
    float qscale;   // scaling * log2(e)
    float* part;    // [n_work][n_kv][g][D + 2]  (o[D], m, l)
    int* counters;  // [batch][n_kv]
};

// Workspace layout shared by lf_decode_workspace_bytes and the kernels: the
// int32 counters [batch][n_kv] sit at offset 0 (a fixed place, so calls with
// different work lists never see another call's partials there), the float
// partials [n_work][n_kv][g][D + 2] follow at a 256-byte boundary.
__host__ __device__ inline int64_t decode_part_offset_bytes(int batch, int n_kv) {
    const int64_t b = static_cast<int64_t>(batch) * n_kv * 4;
    return (b + 255) & ~static_cast<int64_t>(255);
}

__host__ __device__ inline int64_t decode_workspace_total(int batch, int n_kv, int n_q, int head_dim, int n_work) {
    return decode_part_offset_bytes(batch, n_kv) + static_cast<int64_t>(n_work) * n_q * (head_dim + 2) * 4;
}

// Partial record of (item, kv head h, local q head i).
__device__ __forceinline__ float* part_rec(const DecodeParams& p, int item, int h, int i) {
    const int D = p.L.head_dim;
    return p.part + ((static_cast<int64_t>(item) * p.L.n_kv + h) * p.g + i) * (D + 2);
}

// Called by every thread of the workgroup after its partials are stored.
// Returns true in the workgroup that must merge (all threads agree).
__device__ __forceinline__ bool last_split_arrives(const DecodeParams& p, int b, int h, int* flag_lds) {
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int count = p.A.seq_work[2 * b + 1];
        int* ctr = p.counters + b * p.L.n_kv + h;
        const int prev = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        const int last = (prev == count - 1);
        if (last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag_lds = last;
    }
    __syncthreads();
    const bool last = *flag_lds != 0;
    if (last) __threadfence();
    return last;
}

// Merge every item's partial for (b, h) and write out[b][h*g + i][:].
// ``w`` is LDS scratch of ``cap`` floats.  When 2*count*g fits, the (m, l) pairs are
// gathered in one parallel pass, the per-item weights 2^(m_k - M) computed once, and the
// channel loop issues independent loads; otherwise a serial two-pass loop is used.
__device__ inline void merge_partials(const DecodeParams& p, int b, int h, float* w, int cap) {
    const int D = p.L.head_dim;
    const int first = p.A.seq_work[2 * b];
    const int count = p.A.seq_work[2 * b + 1];
    const int n_q = p.A.n_q;
    const int g = p.g;
    const int cg = count * g;
    if (2 * cg <= cap) {
        for (int e = threadIdx.x; e < cg; e += blockDim.x) {
            const float* r = part_rec(p, first + e / g, h, e % g);
            w[e] = r[D];
            w[cg + e] = r[D + 1];
        }
        __syncthreads();
        for (int i = threadIdx.x; i < g; i += blockDim.x) {
            float M = -__builtin_inff();
            for (int k = 0; k < count; ++k) M = fmaxf(M, w[k * g + i]);
            float l = 0.f;
            for (int k = 0; k < count; ++k) {
                const float wk = M == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(w[k * g + i] - M);
                l += wk * w[cg + k * g + i];
                w[k * g + i] = wk;
            }
            w[cg + i] = l;  // (this thread already consumed l of item 0, head i)
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < g * D; idx += blockDim.x) {
            const int i = idx / D;
            const int c = idx % D;
            float o = 0.f;
#pragma unroll 8
            for (int k = 0; k < count; ++k) o += w[k * g + i] * part_rec(p, first + k, h, i)[c];
            const float l = w[cg + i];
            const float val = l > 0.f ? o / l : 0.f;
            store_from_f32(p.A.out, (static_cast<int64_t>(b) * n_q + h * g + i) * D + c, p.A.out_dtype, val);
        }
        return;
    }
    for (int idx = threadIdx.x; idx < g * D; idx += blockDim.x) {
        const int i = idx / D;
        const int c = idx % D;
        float M = -__builtin_inff();
        for (int k = 0; k < count; ++k) M = fmaxf(M, part_rec(p, first + k, h, i)[D]);
        float l = 0.f, o = 0.f;
        if (M != -__builtin_inff()) {
            for (int k = 0; k < count; ++k) {
                const float* r = part_rec(p, first + k, h, i);
                const float wk = __builtin_amdgcn_exp2f(r[D] - M);
                l += r[D + 1] * wk;
                o += r[c] * wk;
            }
        }
        const float val = l > 0.f ? o / l : 0.f;
        store_from_f32(p.A.out, (static_cast<int64_t>(b) * n_q + h * g + i) * D + c, p.A.out_dtype, val);
    }
}

// Load 8 consecutive elements (16-byte aligned for 2-byte types, 32 for fp32) as float.
__device__ __forceinline__ void load8_as_f32(const void* base, int64_t idx, int dt, float* out) {
    if (dt == LF_FP32) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx);
        const float4 c = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + idx + 4);
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = c.x; out[5] = c.y; out[6] = c.z; out[7] = c.w;
        return;
    }
    const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(base) + idx);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint16_t x = static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1)));
        out[k] = dt == LF_BF16 ? bf16_to_f32(x) : f16_to_f32(x);
    }
}

}  // namespace lf
