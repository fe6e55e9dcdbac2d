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
__device__ inline void merge_partials(const DecodeParams& p, int b, int h) {
    const int D = p.L.head_dim;
    const int first = p.A.seq_work[2 * b];
    const int count = p.A.seq_work[2 * b + 1];
    const int n_q = p.A.n_q;
    for (int idx = threadIdx.x; idx < p.g * D; idx += blockDim.x) {
        const int i = idx / D;
        const int c = idx % D;
        float M = -__builtin_inff();
        for (int k = 0; k < count; ++k) M = fmaxf(M, part_rec(p, first + k, h, i)[D]);
        float l = 0.f, o = 0.f;
        if (M != -__builtin_inff()) {
            for (int k = 0; k < count; ++k) {
                const float* r = part_rec(p, first + k, h, i);
                const float w = __builtin_amdgcn_exp2f(r[D] - M);
                l += r[D + 1] * w;
                o += r[c] * w;
            }
        }
        const float val = l > 0.f ? o / l : 0.f;
        const int64_t oi = (static_cast<int64_t>(b) * n_q + h * p.g + i) * D + c;
        store_from_f32(p.A.out, oi, p.A.out_dtype, val);
    }
}

}  // namespace lf
