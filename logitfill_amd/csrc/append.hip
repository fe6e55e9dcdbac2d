// Single-token append to the residual pages, on the device: the one-token commit of a decode
// step (reference src/logitfill/packed/cache.py:48-62 while the page is not full) without a
// host round trip for the write position.  Workgroup b copies sequence b's new Key and Value
// rows of every kv head into row tail_len[b] of its residual page (converted to the residual
// dtype) and then advances tail_len[b]; a full residual page is left untouched (the caller
// flushes full pages before appending).
#include "lf_common.hpp"

namespace lf {
namespace {

struct AppendArgs {
    void* tail_k;
    void* tail_v;
    int tail_dtype, tail_cap;
    int32_t* tail_len;
    const void* k_new;
    const void* v_new;
    int new_dtype;
    int n_kv, head_dim;
};

__global__ __launch_bounds__(256) void append_token_kernel(AppendArgs a) {
    const int b = blockIdx.x;
    const int row = a.tail_len[b];
    __syncthreads();  // every thread has read the position before thread 0 advances it
    if (row < 0 || row >= a.tail_cap) return;
    const int D = a.head_dim;
    for (int e = threadIdx.x; e < a.n_kv * D; e += blockDim.x) {
        const int h = e / D, c = e - h * D;
        const int64_t src = (static_cast<int64_t>(b) * a.n_kv + h) * D + c;
        const int64_t dst = ((static_cast<int64_t>(b) * a.n_kv + h) * a.tail_cap + row) * D + c;
        store_from_f32(a.tail_k, dst, a.tail_dtype, load_as_f32(a.k_new, src, a.new_dtype));
        store_from_f32(a.tail_v, dst, a.tail_dtype, load_as_f32(a.v_new, src, a.new_dtype));
    }
    if (threadIdx.x == 0) a.tail_len[b] = row + 1;
}

}  // namespace

int launch_append_token(void* tail_k, void* tail_v, int tail_dtype, int tail_cap, int32_t* tail_len,
                        const void* k_new, const void* v_new, int new_dtype, int batch, int n_kv, int head_dim,
                        hipStream_t stream) {
    AppendArgs a{tail_k, tail_v, tail_dtype, tail_cap, tail_len, k_new, v_new, new_dtype, n_kv, head_dim};
    hipLaunchKernelGGL(append_token_kernel, dim3(batch), dim3(256), 0, stream, a);
    const hipError_t err = hipGetLastError();
    return err == hipSuccess ? LF_OK : static_cast<int>(err);
}

}  // namespace lf
