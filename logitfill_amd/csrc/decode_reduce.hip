// Cross-split softmax merge (flash-decoding reduce) of the decode partials.
//
// One workgroup per (sequence b, kv head h, local q head i), one thread per
// channel.  The sequence's items are seq_work[b] = (first, count) (the first one also
// covers the tail page and the new token).  With M = max_k m_k over them and w_k = 2^(m_k - M):
//     out[b][h*g + i][c] = sum_k w_k o_k[c] / sum_k w_k l_k,
// the merge of reference.py:44-56's single softmax over all tokens.  Items with
// no tokens carry m = -inf and weigh nothing.
#include <cstddef>
#include <cstring>

#include "decode_common.hpp"

namespace lf {
namespace {

constexpr int kReduceLds = 2048;  // items whose weights are kept in LDS (more: recomputed per channel)
constexpr int kFastItems = 32;    // up to this many items: one round of loads per thread, no LDS
                                  // (at most the 64 lanes of a wave)

struct ReduceParams {
    DecodeParams p;
    int inline_seq;  // 1: seq_inline holds seq_work (at most LF_INLINE_SEQ sequences)
    int pad_;
    int32_t seq_inline[2 * LF_INLINE_SEQ];
};
static_assert(sizeof(ReduceParams) <= 4096, "kernel arguments are limited to 4 KB");

__global__ __launch_bounds__(256) void decode_reduce_kernel(ReduceParams rp) {
    // the argument block and this sequence's inline (first, count), in one round of loads
    const i32x2 seq_arg = prefetch_args_rec2<offsetof(ReduceParams, seq_inline)>(
        static_cast<uint32_t>(offsetof(ReduceParams, seq_inline)) + 8u * min(blockIdx.z, LF_INLINE_SEQ - 1u));
    const DecodeParams& p = rp.p;
    __shared__ float w[kReduceLds];
    __shared__ float red[8];
    const int D = p.L.head_dim;
    const int g = p.g;
    // grid (g, n_kv, batch): no divisions
    const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    // the folded commit: every decode workgroup has read tail_len[b]; advance it once
    if (p.A.commit_new && !p.dense_splits && h == 0 && i == 0 && threadIdx.x == 0)
        const_cast<int32_t*>(p.A.tail_len)[b] += p.q_len;
    const int first = p.dense_splits ? b * p.dense_splits : rp.inline_seq ? seq_arg[0] : p.A.seq_work[2 * b];
    const int count = p.dense_splits ? p.dense_splits : rp.inline_seq ? seq_arg[1] : p.A.seq_work[2 * b + 1];
    const int tid = threadIdx.x;
    const int nw = blockDim.x / kWave;

    if (count <= kFastItems) {
        // One round of loads: lane k of each wave loads item k's (m, l); every thread loads its
        // channels' o of every item.  Each wave then forms the weights in-lane (max and sum by
        // wave reductions) and broadcasts weight k from lane k -- no LDS, no barrier.
        const int lane = tid & (kWave - 1);
        float mk = -__builtin_inff(), lk = 0.f;
        if (lane < count) {
            const float* r = part_rec(p, first + lane, h, i);
            mk = r[D];
            lk = r[D + 1];
        }
        const int c0 = tid;
        float o[kFastItems];
#pragma unroll
        for (int k = 0; k < kFastItems; ++k) o[k] = k < count && c0 < D ? part_rec(p, first + k, h, i)[c0] : 0.f;
        const float M = wave_max(mk);
        const float wk = M == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(mk - M);  // 0 past count
        const float lsum = wave_sum(wk * lk);
        float osum = 0.f;
#pragma unroll
        for (int k = 0; k < kFastItems; ++k) osum = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k)), o[k], osum);
        if (c0 < D)
            store_from_f32(p.A.out, (static_cast<int64_t>(b) * p.A.n_q + h * g + i) * D + c0, p.A.out_dtype,
                           lsum > 0.f ? osum / lsum : 0.f);
        // channels past the first blockDim.x (head_dim 512): the same with the weights kept
        for (int c = c0 + blockDim.x; c < D; c += blockDim.x) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < kFastItems; ++k) {
                const float ok = k < count ? part_rec(p, first + k, h, i)[c] : 0.f;
                acc = fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k)), ok, acc);
            }
            store_from_f32(p.A.out, (static_cast<int64_t>(b) * p.A.n_q + h * g + i) * D + c, p.A.out_dtype,
                           lsum > 0.f ? acc / lsum : 0.f);
        }
        return;
    }

    // M = max over items
    float M = -__builtin_inff();
    for (int k = tid; k < count; k += blockDim.x) M = fmaxf(M, part_rec(p, first + k, h, i)[D]);
    M = wave_max(M);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = M;
    __syncthreads();
    M = red[0];
    for (int k = 1; k < nw; ++k) M = fmaxf(M, red[k]);
    __syncthreads();
    // weights (kept in LDS when they fit) and l = sum w_k l_k
    float l = 0.f;
    for (int k = tid; k < count; k += blockDim.x) {
        const float* r = part_rec(p, first + k, h, i);
        const float wk = M == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(r[D] - M);
        if (k < kReduceLds) w[k] = wk;
        l += wk * r[D + 1];
    }
    l = wave_sum(l);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = l;
    __syncthreads();
    l = 0.f;
    for (int k = 0; k < nw; ++k) l += red[k];
    const int n_lds = count < kReduceLds ? count : kReduceLds;
    for (int c = tid; c < D; c += blockDim.x) {
        float o = 0.f;
#pragma unroll 8
        for (int k = 0; k < n_lds; ++k) o = fmaf(w[k], part_rec(p, first + k, h, i)[c], o);
        for (int k = n_lds; k < count; ++k) {
            const float* r = part_rec(p, first + k, h, i);
            o = fmaf(__builtin_amdgcn_exp2f(r[D] - M), r[c], o);
        }
        const float val = l > 0.f ? o / l : 0.f;
        store_from_f32(p.A.out, (static_cast<int64_t>(b) * p.A.n_q + h * g + i) * D + c, p.A.out_dtype, val);
    }
}

}  // namespace

int launch_decode_reduce(const DecodeParams& p, hipStream_t stream) {
    const int threads = p.L.head_dim < 64 ? 64 : p.L.head_dim > 256 ? 256 : p.L.head_dim;
    ReduceParams rp;
    rp.p = p;
    rp.inline_seq = !p.dense_splits && p.A.seq_work_host != nullptr && p.L.batch <= LF_INLINE_SEQ;
    if (rp.inline_seq) std::memcpy(rp.seq_inline, p.A.seq_work_host, sizeof(int32_t) * 2 * p.L.batch);
    hipLaunchKernelGGL(decode_reduce_kernel, dim3(p.g, p.L.n_kv, p.L.batch), dim3(threads), 0, stream, rp);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
