// Split-K decode: work items and their partial results.
//
// A decode launch covers work items (b, page_begin, page_end, kind) x kv heads.
// Each workgroup produces, for the g = n_q / n_kv query heads of its kv head,
// a partial (m, l, o[D]) over its tokens: m the running max of the log2-domain
// scores, l = sum 2^(s - m), o = sum 2^(s - m) v.  decode_reduce_kernel
// (decode_reduce.hip) then merges each sequence's partials into the output
// (the flash-decoding reduce).
#pragma once

#include "lf_common.hpp"

namespace lf {

struct DecodeParams {
    lf_packed_layer L;
    lf_decode_args A;
    int g;          // query rows per kv head: (n_q / n_kv) * q_len, row = head * q_len + token
    int q_len;      // new query tokens per sequence (A.n_q counts rows: n_q * q_len)
    float qscale;   // scaling * log2(e)
    float* part;    // [n_work][n_kv][g][D + 2]  (o[D], m, l)
    int dense_splits;  // > 0: items b * dense_splits .. + dense_splits - 1 are sequence b's
                       // (the dense comparator); 0: A.seq_work lists them
};

// Workspace layout shared by lf_decode_workspace_bytes and the kernels: the float
// partials [n_work][n_kv][g][D + 2] from offset 0.  Nothing needs initialising.
__host__ __device__ inline int64_t decode_workspace_total(int n_q, int head_dim, int n_work) {
    return static_cast<int64_t>(n_work) * n_q * (head_dim + 2) * 4;
}

// Partial record of (item, kv head h, local q head i).
__device__ __forceinline__ float* part_rec(const DecodeParams& p, int item, int h, int i) {
    const int D = p.L.head_dim;
    return p.part + ((static_cast<int64_t>(item) * p.L.n_kv + h) * p.g + i) * (D + 2);
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

// Bring the kernel's argument block (ceil(Bytes / 64) whole 64-byte lines: the last may reach into
// the hidden arguments that follow the explicit ones in the kernarg segment) into the scalar data
// cache with one round of loads, issued from one asm
// statement so that no compiler wait splits it.  The compiler reads argument fields lazily, a small
// load and a wait at a time where register pressure makes it re-read them; with the block already
// cached each of those waits is a cache hit instead of a memory round trip.  The loaded values are
// discarded (s40..s55 are clobbered); the asm declares no memory clobber, so loads of read-only
// data may still be scalar loads.
#define LF_ARG_LINE(off) "s_load_dwordx16 s[40:55], %[kp], " #off "\n\t"
#define LF_ARG_LINES6 LF_ARG_LINE(0) LF_ARG_LINE(64) LF_ARG_LINE(128) LF_ARG_LINE(192) LF_ARG_LINE(256) LF_ARG_LINE(320)
#define LF_ARG_CLOBBERS "s40", "s41", "s42", "s43", "s44", "s45", "s46", "s47", "s48", "s49", "s50", "s51", \
    "s52", "s53", "s54", "s55"
#define LF_ARG_LINES(lines)                                                                          \
    LF_ARG_LINES6 LF_ARG_LINE(384) LF_ARG_LINE(448) LF_ARG_LINE(512) LF_ARG_LINE(576)
// One asm statement per line count (6..10), with ``EXTRA`` loads before the single wait.
#define LF_PREFETCH(EXTRA, ...)                                                                      \
    if constexpr (lines == 6)                                                                        \
        asm volatile(LF_ARG_LINES6 EXTRA "s_waitcnt lgkmcnt(0)" __VA_ARGS__ : LF_ARG_CLOBBERS);         \
    else if constexpr (lines == 7)                                                                   \
        asm volatile(LF_ARG_LINES6 LF_ARG_LINE(384) EXTRA "s_waitcnt lgkmcnt(0)" __VA_ARGS__ : LF_ARG_CLOBBERS); \
    else if constexpr (lines == 8)                                                                   \
        asm volatile(LF_ARG_LINES6 LF_ARG_LINE(384) LF_ARG_LINE(448) EXTRA "s_waitcnt lgkmcnt(0)"       \
                     __VA_ARGS__ : LF_ARG_CLOBBERS);                                                 \
    else if constexpr (lines == 9)                                                                   \
        asm volatile(LF_ARG_LINES6 LF_ARG_LINE(384) LF_ARG_LINE(448) LF_ARG_LINE(512) EXTRA            \
                     "s_waitcnt lgkmcnt(0)" __VA_ARGS__ : LF_ARG_CLOBBERS);                          \
    else                                                                                             \
        asm volatile(LF_ARG_LINES(10) EXTRA "s_waitcnt lgkmcnt(0)" __VA_ARGS__ : LF_ARG_CLOBBERS);
template <int Bytes>
__device__ __forceinline__ void prefetch_args() {
    constexpr int lines = (Bytes + 63) / 64;
    static_assert(lines >= 6 && lines <= 10, "prefetch_args: add the line count of this argument block");
    const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    LF_PREFETCH("", ::[kp] "s"(kp))
}

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
// prefetch_args of the first ``Bytes`` bytes plus one record of the argument block at byte offset
// ``off`` (uniform), loaded in the same round and returned: a plan entry that travels in the
// kernel arguments arrives with them instead of one dependent memory round trip later.
template <int Bytes>
__device__ __forceinline__ i32x4 prefetch_args_rec4(uint32_t off) {
    constexpr int lines = (Bytes + 63) / 64;
    static_assert(lines >= 6 && lines <= 10, "prefetch_args: add the line count of this argument block");
    const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    i32x4 rec;
    LF_PREFETCH("s_load_dwordx4 %[rec], %[kp], %[off]\n\t", : [rec] "=s"(rec) : [kp] "s"(kp), [off] "s"(off))
    return rec;
}
template <int Bytes>
__device__ __forceinline__ i32x2 prefetch_args_rec2(uint32_t off) {
    constexpr int lines = (Bytes + 63) / 64;
    static_assert(lines >= 6 && lines <= 10, "prefetch_args: add the line count of this argument block");
    const auto kp = __builtin_amdgcn_kernarg_segment_ptr();
    i32x2 rec;
    LF_PREFETCH("s_load_dwordx2 %[rec], %[kp], %[off]\n\t", : [rec] "=s"(rec) : [kp] "s"(kp), [off] "s"(off))
    return rec;
}
#undef LF_PREFETCH
#undef LF_ARG_LINES
#undef LF_ARG_CLOBBERS
#undef LF_ARG_LINES6
#undef LF_ARG_LINE

// The commit folded into the decode (lf_decode_args.commit_new): the workgroup that owns
// sequence b's residual for kv head h (row tile 0) copies the new rows into the tail buffer at
// the device-side tail length every decode workgroup reads; nothing in the launch reads those
// rows (the residual pass takes the new tokens from k_new / v_new).  The reduce kernel then
// advances the length, after every decode workgroup has read it.
__device__ __forceinline__ void commit_new_rows(const DecodeParams& p, int b, int h, int tid, int nthreads) {
    const lf_decode_args& A = p.A;
    const int tl = A.tail_len[b];
    const int D = p.L.head_dim, q_len = p.q_len;
    if (tl < 0 || tl + q_len > A.tail_cap) return;  // the host keeps it below; bounds safety
    for (int e = tid; e < q_len * D; e += nthreads) {
        const int t = e / D, c = e - t * D;
        const int64_t bh = static_cast<int64_t>(b) * p.L.n_kv + h;
        const int64_t src = (bh * q_len + t) * D + c;
        const int64_t dst = (bh * A.tail_cap + tl + t) * D + c;
        store_from_f32(const_cast<void*>(A.tail_k), dst, A.tail_dtype, load_as_f32(A.k_new, src, A.new_dtype));
        store_from_f32(const_cast<void*>(A.tail_v), dst, A.tail_dtype, load_as_f32(A.v_new, src, A.new_dtype));
    }
}

// Merge the partials of every sequence into ``out`` (enqueued after a decode kernel).  With the
// host copy of seq_work and at most LF_INLINE_SEQ sequences, the (first, count) pairs go into
// the reduce kernel's arguments.
int launch_decode_reduce(const DecodeParams& p, hipStream_t stream);

}  // namespace lf
