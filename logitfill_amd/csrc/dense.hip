// BF16 dense split-K decode attention (placeholder: not yet built).
#include "decode_common.hpp"

namespace lf {

int64_t dense_workspace_bytes(int batch, int n_kv, int n_q, int head_dim, int tokens, int tokens_per_split) {
    const int64_t splits = (tokens + tokens_per_split - 1) / tokens_per_split;
    return static_cast<int64_t>(batch) * n_q * splits * (head_dim + 2) * 4 + 256 +
           static_cast<int64_t>(batch) * n_kv * 4;
}

int launch_dense_decode(const void*, const void*, const void*, int, int, int, int, int, int64_t, int64_t,
                        int64_t, float, void*, int, void*, hipStream_t) {
    return LF_E_UNSUPPORTED;
}

}  // namespace lf
