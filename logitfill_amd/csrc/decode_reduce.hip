// Cross-split softmax merge (flash-decoding reduce) of the decode partials.
//
// One workgroup per (sequence b, kv head h, local q head i), one thread per
// channel.  The sequence's items are seq_work[b] = (first, count) (the first one also
// covers the tail page and the new token).  With M = max_k m_k over them and w_k = 2^(m_k - M):
//     out[b][h*g + i][c] = sum_k w_k o_k[c] / sum_k w_k l_k,
// the merge of reference.py:44-56's single softmax over all tokens.  Items with
// no tokens carry m = -inf and weigh nothing.
#include "decode_common.hpp"

namespace lf {
namespace {

constexpr int kReduceLds = 2048;  // items whose weights are kept in LDS (more: recomputed per channel)
constexpr int kFastItems = 16;    // up to this many items: one round of loads per thread, no LDS

__global__ __launch_bounds__(256) void decode_reduce_kernel(DecodeParams p) {
    __shared__ float w[kReduceLds];
    __shared__ float red[8];
    const int D = p.L.head_dim;
    const int g = p.g;
    const int i = blockIdx.x % g;
    const int h = (blockIdx.x / g) % p.L.n_kv;
    const int b = blockIdx.x / (g * p.L.n_kv);
    const int first = p.dense_splits ? b * p.dense_splits : p.A.seq_work[2 * b];
    const int count = p.dense_splits ? p.dense_splits : p.A.seq_work[2 * b + 1];
    const int tid = threadIdx.x;
    const int nw = blockDim.x / kWave;

    if (count <= kFastItems) {
        // Every thread loads all items' (m, l) -- the same addresses across the workgroup --
        // and its channels' o, all before the first use: one load latency per channel pass.
        float m[kFastItems], l[kFastItems];
#pragma unroll
        for (int k = 0; k < kFastItems; ++k) {
            m[k] = -__builtin_inff();
            l[k] = 0.f;
            if (k < count) {
                const float* r = part_rec(p, first + k, h, i);
                m[k] = r[D];
                l[k] = r[D + 1];
            }
        }
        for (int c = tid; c < D; c += blockDim.x) {
            float o[kFastItems];
#pragma unroll
            for (int k = 0; k < kFastItems; ++k) o[k] = k < count ? part_rec(p, first + k, h, i)[c] : 0.f;
            float M = m[0];
#pragma unroll
            for (int k = 1; k < kFastItems; ++k) M = fmaxf(M, m[k]);
            float lsum = 0.f, osum = 0.f;
            if (M != -__builtin_inff()) {
#pragma unroll
                for (int k = 0; k < kFastItems; ++k) {
                    const float wk = __builtin_amdgcn_exp2f(m[k] - M);  // 0 for the items past count
                    lsum = fmaf(wk, l[k], lsum);
                    osum = fmaf(wk, o[k], osum);
                }
            }
            store_from_f32(p.A.out, (static_cast<int64_t>(b) * p.A.n_q + h * g + i) * D + c, p.A.out_dtype,
                           lsum > 0.f ? osum / lsum : 0.f);
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
    hipLaunchKernelGGL(decode_reduce_kernel, dim3(p.L.batch * p.L.n_kv * p.g), dim3(threads), 0, stream, p);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
