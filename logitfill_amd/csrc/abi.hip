// extern "C" entry points of liblogitfill_amd.so (declared in include/logitfill_amd.h).
//
// Validation happens here, before anything is enqueued: a negative LF_E_* code
// means nothing ran.  The library keeps no mutable state and allocates nothing.
#include "decode_common.hpp"

namespace lf {
int launch_pack_pages(const lf_packed_layer& L, const void* k_src, const void* v_src, int src_dtype,
                      int64_t sb, int64_t sh, int64_t st, const int32_t* jobs, int n_jobs,
                      hipStream_t stream);
int launch_pack_pages_multi(const lf_packed_layer* layers_dev, const lf_packed_layer* layers_host,
                            const lf_pack_source* srcs_dev, const lf_pack_source* srcs_host, int n_layers,
                            int src_dtype, const int32_t* jobs, int n_jobs, hipStream_t stream);
int launch_decode_valu(const DecodeParams& p, hipStream_t stream);
int launch_decode_mfma(const DecodeParams& p, hipStream_t stream, bool* handled);
int launch_dequantize(const lf_packed_layer& L, int b, int tokens, float* k_out, float* v_out,
                      hipStream_t stream);
int launch_dense_decode(const void* query, const void* k, const void* v, int batch, int n_q, int n_kv,
                        int head_dim, int tokens, int64_t sb, int64_t sh, int64_t st, float scaling,
                        void* out, int tokens_per_split, void* workspace, hipStream_t stream);
int64_t dense_workspace_bytes(int batch, int n_kv, int n_q, int head_dim, int tokens, int tokens_per_split);
int launch_asymmetric_codes(const void* x, int dtype, int64_t n_groups, int group, int bits, int32_t* codes,
                            float* scale, float* lo, hipStream_t stream);
int launch_pack_ints(const int32_t* codes, int64_t rows, int n, int bits, int32_t* words, hipStream_t stream);
int launch_unpack_ints(const int32_t* words, int64_t rows, int n_words, int count, int bits, int32_t* codes,
                       hipStream_t stream);
int launch_append_token(void* tail_k, void* tail_v, int tail_dtype, int tail_cap, int32_t* tail_len,
                        const void* k_new, const void* v_new, int new_dtype, int batch, int n_kv, int head_dim,
                        hipStream_t stream);
}  // namespace lf

namespace {

bool valid_dtype(int32_t d) { return d == LF_BF16 || d == LF_FP16 || d == LF_FP32; }

// Shape and pointer checks shared by every entry point that reads a layer.
// ``need_k`` / ``need_v``: validate the Key tiers / the Value arrays.
int32_t check_layer(const lf_packed_layer* L, bool need_k = true, bool need_v = true) {
    if (!L) return LF_E_NULL;
    if (L->batch <= 0 || L->n_kv <= 0 || L->head_dim <= 0 || L->page_size <= 0 || L->k_group <= 0)
        return LF_E_SHAPE;
    if (L->page_size % L->k_group != 0) return LF_E_SHAPE;
    if (L->cap_tokens < 0 || L->cap_kgroups < 0) return LF_E_SHAPE;
    if (static_cast<int64_t>(L->cap_kgroups) * L->k_group < L->cap_tokens) return LF_E_SHAPE;
    if (need_k) {
        int wsum = 0;
        for (int t = 0; t < 4; ++t) {
            if (L->k_width[t] < 0 || L->k_width[t] > L->head_dim) return LF_E_SHAPE;
            wsum += L->k_width[t];
            if (L->k_width[t] > 0 && (!L->tier_index[t] || !L->tier_count[t])) return LF_E_NULL;
        }
        if (wsum < L->head_dim) return LF_E_SHAPE;  // every channel has a tier
        for (int t = 0; t < 3; ++t) {
            const int per = 32 / (2 << t);
            if (L->k_words[t] != (L->k_width[t] + per - 1) / per) return LF_E_SHAPE;
            if (L->k_width[t] > 0 && (!L->k_code[t] || !L->k_scale[t] || !L->k_min[t])) return LF_E_NULL;
        }
        if (L->k_width[3] > 0 && !L->k_value16) return LF_E_NULL;
    }
    if (need_v) {
        if (L->bit_v >= 16) {
            if (!L->v_value16) return LF_E_NULL;
        } else {
            if (L->bit_v != 2 && L->bit_v != 4 && L->bit_v != 8) return LF_E_SHAPE;
            if (L->v_group <= 0 || L->head_dim % L->v_group != 0) return LF_E_SHAPE;
            if (L->v_groups != L->head_dim / L->v_group) return LF_E_SHAPE;
            if (L->v_words != (L->head_dim * L->bit_v + 31) / 32) return LF_E_SHAPE;  // last word padded
            if (!L->v_code || !L->v_scale || !L->v_min) return LF_E_NULL;
        }
    }
    return LF_OK;
}

}  // namespace

namespace lf {

// Checks shared by the decode entry points, then the launch with ``workspace`` (at least
// ``workspace_bytes``) as the split-K partials.  The args' own workspace fields are not read.
int32_t decode_checked(const lf_packed_layer* layer, const lf_decode_args* args, void* workspace,
                       int64_t workspace_bytes, void* stream) {
    const int32_t st = check_layer(layer);
    if (st != LF_OK) return st;
    if (!args) return LF_E_NULL;
    const lf_decode_args& A = *args;
    if (!A.query || !A.out || !A.work || !A.seq_work || !workspace || !A.tail_len) return LF_E_NULL;
    if ((A.k_new == nullptr) != (A.v_new == nullptr)) return LF_E_NULL;
    if (!valid_dtype(A.q_dtype) || !valid_dtype(A.out_dtype) || !valid_dtype(A.tail_dtype)) return LF_E_DTYPE;
    if (A.k_new && !valid_dtype(A.new_dtype)) return LF_E_DTYPE;
    if (A.n_q <= 0 || A.n_q % layer->n_kv != 0) return LF_E_SHAPE;
    if (A.q_len < 0) return LF_E_SHAPE;
    const int q_len = A.q_len > 1 ? A.q_len : 1;
    // q_len new tokens: the kernels serve n_q * q_len query rows (row = head * q_len + token)
    const int64_t rows = static_cast<int64_t>(A.n_q) * q_len;
    if (rows > (1 << 20)) return LF_E_SHAPE;
    // rows per kv head: any number (the kernels tile them across workgroups)
    const int g = static_cast<int>(rows / layer->n_kv);
    if (layer->bit_v != 2) return LF_E_UNSUPPORTED;  // as reference.py:62
    const int D = layer->head_dim;
    if (D < 8 || D > 1024 || (D & (D - 1)) != 0) return LF_E_UNSUPPORTED;  // as kernel.cu:224-230
    if (layer->v_groups > 64) return LF_E_UNSUPPORTED;
    if (A.tail_cap < 0 || A.tail_cap > layer->page_size) return LF_E_SHAPE;
    if (A.tail_cap > 0 && (!A.tail_k || !A.tail_v)) return LF_E_NULL;
    if (A.n_work <= 0 || static_cast<int64_t>(A.n_work) * layer->n_kv > 0x7fffffff) return LF_E_SHAPE;
    if (workspace_bytes < lf_decode_workspace_bytes(static_cast<int32_t>(rows), D, A.n_work)) return LF_E_WORKSPACE;
    if (A.kernel < 0 || A.kernel > 2) return LF_E_SHAPE;
    if (A.commit_new != 0 && A.commit_new != 1) return LF_E_SHAPE;
    if (A.commit_new && (!A.k_new || A.tail_cap < q_len)) return LF_E_SHAPE;  // rows to append, room for them

    DecodeParams p;
    p.L = *layer;
    p.A = A;
    p.A.n_q = static_cast<int32_t>(rows);
    p.A.workspace = workspace;
    p.A.workspace_bytes = workspace_bytes;
    p.g = g;
    p.q_len = q_len;
    p.qscale = A.scaling * kLog2e;
    p.part = static_cast<float*>(workspace);
    p.dense_splits = 0;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (A.kernel != 1) {
        bool handled = false;
        const int r = launch_decode_mfma(p, s, &handled);
        if (handled || A.kernel == 2) return handled ? r : LF_E_UNSUPPORTED;
    }
    return launch_decode_valu(p, s);
}

}  // namespace lf

extern "C" {

int32_t lf_abi_version(void) { return LF_ABI_VERSION; }

const char* lf_build_info(void) {
    return "logitfill_amd " __DATE__ " " __TIME__ " gfx950 wave64";
}

const char* lf_status_string(int32_t status) {
    switch (status) {
        case LF_OK: return "ok";
        case LF_E_NULL: return "a required pointer is NULL";
        case LF_E_SHAPE: return "inconsistent or unsupported shape";
        case LF_E_UNSUPPORTED: return "configuration not implemented";
        case LF_E_WORKSPACE: return "workspace too small";
        case LF_E_DTYPE: return "unknown dtype code";
        default: break;
    }
    return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown status";
}

// Page jobs are the grid's x dimension (n_jobs workgroups of up to 512 threads): 2^21 jobs keep
// its work-items far below the 2^32 of a dimension.
constexpr int32_t kMaxPackJobs = 1 << 21;

int32_t lf_pack_pages(const lf_packed_layer* layer, const void* k_src, const void* v_src, int32_t src_dtype,
                      int64_t src_stride_b, int64_t src_stride_h, int64_t src_stride_t,
                      const int32_t* jobs, int32_t n_jobs, void* stream) {
    const int32_t st = check_layer(layer);
    if (st != LF_OK) return st;
    if (!valid_dtype(src_dtype)) return LF_E_DTYPE;
    if (n_jobs < 0 || n_jobs > kMaxPackJobs) return LF_E_SHAPE;
    if (n_jobs == 0) return LF_OK;
    if (!k_src || !v_src || !jobs) return LF_E_NULL;
    if (layer->page_size > 1024 || layer->head_dim > 1024) return LF_E_SHAPE;
    return lf::launch_pack_pages(*layer, k_src, v_src, src_dtype, src_stride_b, src_stride_h, src_stride_t,
                                 jobs, n_jobs, static_cast<hipStream_t>(stream));
}

int32_t lf_pack_pages_multi(const lf_packed_layer* layers_dev, const lf_packed_layer* layers_host,
                            const lf_pack_source* srcs_dev, const lf_pack_source* srcs_host, int32_t n_layers,
                            int32_t src_dtype, const int32_t* jobs, int32_t n_jobs, void* stream) {
    if (n_layers < 0 || n_jobs < 0 || n_jobs > kMaxPackJobs) return LF_E_SHAPE;
    if (n_jobs == 0 || n_layers == 0) return n_jobs == 0 ? LF_OK : LF_E_SHAPE;
    if (!layers_dev || !layers_host || !srcs_dev || !srcs_host || !jobs) return LF_E_NULL;
    if (!valid_dtype(src_dtype)) return LF_E_DTYPE;
    for (int32_t i = 0; i < n_layers; ++i) {
        const int32_t st = check_layer(&layers_host[i]);
        if (st != LF_OK) return st;
        if (!srcs_host[i].k || !srcs_host[i].v) return LF_E_NULL;
    }
    return lf::launch_pack_pages_multi(layers_dev, layers_host, srcs_dev, srcs_host, n_layers, src_dtype, jobs,
                                       n_jobs, static_cast<hipStream_t>(stream));
}

int32_t lf_plan_decode(const int32_t* hist_pages, int32_t batch, int32_t pages_per_split, int32_t residual_pages,
                       int32_t* work_out, int32_t work_cap, int32_t* seq_work_out) {
    if (!hist_pages || !work_out || !seq_work_out) return LF_E_NULL;
    if (batch <= 0 || pages_per_split <= 0 || residual_pages < 0) return LF_E_SHAPE;
    // Sequence b's work is its residual (tail page + new token), costed as ``residual_pages``
    // pages, followed by its packed pages.  It is cut into ceil(work / pages_per_split) items
    // of equal work; the first item takes the residual and the pages left in its share.
    int32_t n = 0;
    for (int32_t b = 0; b < batch; ++b) {
        const int32_t pages = hist_pages[b];
        if (pages < 0) return LF_E_SHAPE;
        const int32_t first = n;
        const int64_t work = static_cast<int64_t>(pages) + residual_pages;
        const int64_t items = pages == 0 ? 1 : (work + pages_per_split - 1) / pages_per_split;
        for (int64_t k = 0; k < items; ++k) {
            const int64_t w0 = k * work / items, w1 = (k + 1) * work / items;
            const int32_t p0 = static_cast<int32_t>(w0 > residual_pages ? w0 - residual_pages : 0);
            const int32_t p1 = static_cast<int32_t>(w1 > residual_pages ? w1 - residual_pages : 0);
            if (k > 0 && p1 == p0) continue;
            if (n >= work_cap) return LF_E_WORKSPACE;
            work_out[4 * n + 0] = b;
            work_out[4 * n + 1] = p0;
            work_out[4 * n + 2] = p1;
            work_out[4 * n + 3] = k > 0 ? 0 : p1 > p0 ? 2 : 1;
            ++n;
        }
        seq_work_out[2 * b + 0] = first;
        seq_work_out[2 * b + 1] = n - first;
    }
    return n;
}

int64_t lf_decode_workspace_bytes(int32_t n_q, int32_t head_dim, int32_t n_work) {
    if (n_q <= 0 || head_dim <= 0 || n_work < 0) return LF_E_SHAPE;
    return lf::decode_workspace_total(n_q, head_dim, n_work);
}

int32_t lf_decode_attention(const lf_packed_layer* layer, const lf_decode_args* args, void* stream) {
    return lf::decode_checked(layer, args, args ? args->workspace : nullptr, args ? args->workspace_bytes : 0,
                              stream);
}

int32_t lf_dequantize(const lf_packed_layer* layer, int32_t b, int32_t tokens, float* k_out, float* v_out,
                      void* stream) {
    if (!k_out && !v_out) return LF_E_NULL;
    const int32_t st = check_layer(layer, k_out != nullptr, v_out != nullptr);
    if (st != LF_OK) return st;
    if (b < 0 || b >= layer->batch || tokens < 0 || tokens > layer->cap_tokens) return LF_E_SHAPE;
    if (tokens == 0) return LF_OK;
    return lf::launch_dequantize(*layer, b, tokens, k_out, v_out, static_cast<hipStream_t>(stream));
}

int64_t lf_dense_decode_workspace_bytes(int32_t batch, int32_t n_kv, int32_t n_q, int32_t head_dim,
                                        int32_t tokens, int32_t tokens_per_split) {
    return lf::dense_workspace_bytes(batch, n_kv, n_q, head_dim, tokens, tokens_per_split);
}

int32_t lf_dense_decode(const void* query, const void* k, const void* v, int32_t batch, int32_t n_q,
                        int32_t n_kv, int32_t head_dim, int32_t tokens, int64_t kv_stride_b,
                        int64_t kv_stride_h, int64_t kv_stride_t, float scaling, void* out,
                        int32_t tokens_per_split, void* workspace, int64_t workspace_bytes, void* stream) {
    if (!query || !k || !v || !out || !workspace) return LF_E_NULL;
    if (batch <= 0 || n_kv <= 0 || n_q <= 0 || n_q % n_kv != 0 || tokens <= 0) return LF_E_SHAPE;
    if (n_q / n_kv > 8) return LF_E_UNSUPPORTED;
    if (head_dim != 128) return LF_E_UNSUPPORTED;
    if (tokens_per_split <= 0 || tokens_per_split % 128 != 0) return LF_E_SHAPE;
    if (workspace_bytes < lf::dense_workspace_bytes(batch, n_kv, n_q, head_dim, tokens, tokens_per_split))
        return LF_E_WORKSPACE;
    return lf::launch_dense_decode(query, k, v, batch, n_q, n_kv, head_dim, tokens, kv_stride_b, kv_stride_h,
                                   kv_stride_t, scaling, out, tokens_per_split, workspace,
                                   static_cast<hipStream_t>(stream));
}

int32_t lf_append_token(void* tail_k, void* tail_v, int32_t tail_dtype, int32_t tail_cap, int32_t* tail_len,
                        const void* k_new, const void* v_new, int32_t new_dtype, int32_t batch, int32_t n_kv,
                        int32_t head_dim, void* stream) {
    if (!valid_dtype(tail_dtype) || !valid_dtype(new_dtype)) return LF_E_DTYPE;
    if (batch <= 0 || n_kv <= 0 || head_dim <= 0 || tail_cap <= 0) return LF_E_SHAPE;
    if (!tail_k || !tail_v || !tail_len || !k_new || !v_new) return LF_E_NULL;
    return lf::launch_append_token(tail_k, tail_v, tail_dtype, tail_cap, tail_len, k_new, v_new, new_dtype, batch,
                                   n_kv, head_dim, static_cast<hipStream_t>(stream));
}

int32_t lf_asymmetric_codes(const void* x, int32_t dtype, int64_t n_groups, int32_t group, int32_t bits,
                            int32_t* codes, float* scale, float* lo, void* stream) {
    if (!valid_dtype(dtype)) return LF_E_DTYPE;
    if (n_groups < 0 || group <= 0 || bits < 1 || bits > 16) return LF_E_SHAPE;
    if (n_groups == 0) return LF_OK;
    if (!x || !codes || !scale || !lo) return LF_E_NULL;
    if (n_groups > (static_cast<int64_t>(1) << 33)) return LF_E_SHAPE;
    return lf::launch_asymmetric_codes(x, dtype, n_groups, group, bits, codes, scale, lo,
                                       static_cast<hipStream_t>(stream));
}

int32_t lf_pack_ints(const int32_t* codes, int64_t rows, int32_t n, int32_t bits, int32_t* words, void* stream) {
    if (rows < 0 || n < 0 || bits <= 0 || bits > 32) return LF_E_SHAPE;
    if (rows == 0 || n == 0) return LF_OK;
    if (!codes || !words) return LF_E_NULL;
    const int per = 32 / bits;
    if (rows * ((n + per - 1) / per) > (static_cast<int64_t>(1) << 40)) return LF_E_SHAPE;
    return lf::launch_pack_ints(codes, rows, n, bits, words, static_cast<hipStream_t>(stream));
}

int32_t lf_unpack_ints(const int32_t* words, int64_t rows, int32_t n_words, int32_t count, int32_t bits,
                       int32_t* codes, void* stream) {
    if (rows < 0 || n_words < 0 || count < 0 || bits <= 0 || bits > 32) return LF_E_SHAPE;
    if (static_cast<int64_t>(count) > static_cast<int64_t>(n_words) * (32 / bits)) return LF_E_SHAPE;
    if (rows == 0 || count == 0) return LF_OK;
    if (!words || !codes) return LF_E_NULL;
    if (rows * count > (static_cast<int64_t>(1) << 40)) return LF_E_SHAPE;
    return lf::launch_unpack_ints(words, rows, n_words, count, bits, codes, static_cast<hipStream_t>(stream));
}

}  // extern "C"
