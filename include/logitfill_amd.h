/*
 * logitfill_amd -- C ABI of the MI355X (gfx950) packed KV decode path.
 *
 * Replaces the reference's single native entry point, the pybind11/torch
 * function ``logitfill_decode`` (reference src/logitfill/packed/kernel.cu:198-284,
 * JIT-loaded by src/logitfill/packed/kernel_loader.py:14-35), and moves the
 * reference's Python/torch page packer (src/logitfill/packed/layout.py:71-129,
 * called from src/logitfill/packed/cache.py:64-81) onto the device.
 *
 * Conventions
 *  - Plain C: device pointers, sizes and strides only; no torch types.
 *  - The caller owns every buffer, including outputs and workspaces; the
 *    library never allocates device memory.  Its only mutable global state is
 *    the per-device address of the scratch array of
 *    lf_decode_attention_noalloc, looked up once per device under a lock; every
 *    entry point is re-entrant and may be called from several host threads.
 *  - ``stream`` is a hipStream_t passed as ``void*`` (NULL = default stream).
 *    Nothing synchronises inside; all work is enqueued on ``stream``.
 *  - Return value: 0 = success; negative = argument/shape error (LF_E_*),
 *    nothing enqueued; positive = hipError_t of a failed launch.
 *  - Float16 data is passed as ``uint16_t`` bit patterns.
 */
#ifndef LOGITFILL_AMD_H
#define LOGITFILL_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LF_ABI_VERSION 8

/* Element types of query / residual / output tensors. */
enum lf_dtype { LF_BF16 = 0, LF_FP16 = 1, LF_FP32 = 2 };

/* Status codes (negative: rejected before launch). */
enum lf_status {
    LF_OK = 0,
    LF_E_NULL = -1,          /* a required pointer is NULL                     */
    LF_E_SHAPE = -2,         /* sizes inconsistent or out of supported range    */
    LF_E_UNSUPPORTED = -3,   /* valid but not implemented (e.g. bit_v != 2)     */
    LF_E_WORKSPACE = -4,     /* workspace too small                             */
    LF_E_DTYPE = -5          /* unknown dtype code                              */
};

/*
 * One layer's packed history for ``batch`` sequences, in the reference byte
 * layout (src/logitfill/packed/cache.py:64-81 and layout.py:71-129) with a
 * capacity stride on the growing axis:
 *
 *   k_code[t]   int32 [batch][n_kv][cap_tokens][k_words[t]]     t = 0,1,2 (int2/int4/int8)
 *   k_scale[t]  fp16  [batch][n_kv][k_width[t]][cap_kgroups]    (page/group index innermost)
 *   k_min[t]    fp16  [batch][n_kv][k_width[t]][cap_kgroups]
 *   k_value16   fp16  [batch][n_kv][cap_tokens][k_width[3]]     (fp16 tier)
 *   v_code      int32 [batch][n_kv][cap_tokens][v_words]        (bit_v < 16; v_words =
 *                                                                ceil(head_dim * bit_v / 32),
 *                                                                the last word zero padded
 *                                                                as layout.py:27-29 pads)
 *   v_scale     fp16  [batch][n_kv][cap_tokens][v_groups]       (bit_v < 16)
 *   v_min       fp16  [batch][n_kv][cap_tokens][v_groups]       (bit_v < 16)
 *   v_value16   fp16  [batch][n_kv][cap_tokens][head_dim]       (bit_v >= 16)
 *
 * Sequence b's reference tensors are the slices [b][:, :hist_len, :] (codes,
 * values) and [b][:, :, :hist_len/k_group] (Key scale/min).  The tier table
 * (src/logitfill/packed/layout.py:49-68) is passed as ``tier_index[t]``
 * int32 [n_kv][k_width[t]] (ascending channel ids, zero padded) and
 * ``tier_count[t]`` int32 [n_kv].  Pointers of empty tiers may be NULL.
 *
 * Beside the reference arrays, a layer whose Key group is the page (k_group == page_size)
 * may carry a page-major copy of the integer tiers' Key scales and mins, the form the
 * matrix-core decode kernel reads (one contiguous block per page instead of one fp16 pair
 * per slot and page, each in a cache line of its own):
 *
 *   k_sm_page   fp16  [batch][n_kv][cap_kgroups][16 * nb]
 *
 * nb = 4 * (2 * ceil(k_words[0] / 4) + ceil(k_words[1] / 4) + ceil(ceil(k_words[2] / 2) / 4))
 * blocks of 8 slots, tier by tier; block i holds 8 scales then 8 mins.  The slot order inside a
 * tier's blocks is the decode kernel's code-unpack order (logitfill_amd/csrc/lf_common.hpp,
 * sm_slot / sm_place); positions that are no channel of the head hold scale 1.0 and min 0.0.
 * Every packer writes it when the pointer is not NULL (the values are bit-identical to the
 * reference arrays'); decode takes the matrix-core kernel only when it is present.
 */
typedef struct lf_packed_layer {
    int32_t*  k_code[3];
    uint16_t* k_scale[3];
    uint16_t* k_min[3];
    uint16_t* k_value16;
    int32_t*  v_code;
    uint16_t* v_scale;
    uint16_t* v_min;
    uint16_t* v_value16;
    const int32_t* tier_index[4];
    const int32_t* tier_count[4];
    int32_t batch, n_kv, head_dim;
    int32_t cap_tokens, cap_kgroups;
    int32_t page_size, k_group, v_group, bit_v;
    int32_t k_width[4];
    int32_t k_words[3];
    int32_t v_words, v_groups;
    uint16_t* k_sm_page;              /* page-major Key scale/min copy, or NULL (see above) */
} lf_packed_layer;

/* ABI version (LF_ABI_VERSION) and a static build string. */
int32_t lf_abi_version(void);
const char* lf_build_info(void);
const char* lf_status_string(int32_t status);

/*
 * Page compress.  Replaces quantize_key_page + quantize_value_page + the
 * history concatenation of _LayerStore._flush
 * (reference src/logitfill/packed/layout.py:71-129, cache.py:64-81).
 *
 * Packs ``n_jobs`` pages (at most 2^21 per call, else LF_E_SHAPE).  ``jobs``
 * is a DEVICE int32 array [n_jobs][3] of
 * (b, src_token0, dst_page): the page is rows src_token0 .. src_token0 +
 * page_size - 1 of sequence b of ``k_src``/``v_src`` (element strides
 * src_stride_b/h/t, channel stride 1, dtype ``src_dtype``) and is written as
 * page ``dst_page`` of sequence b of ``layer``.  Codes, scales and mins are
 * bit-exact with the reference packer on finite inputs.
 */
int32_t lf_pack_pages(const lf_packed_layer* layer,
                      const void* k_src, const void* v_src, int32_t src_dtype,
                      int64_t src_stride_b, int64_t src_stride_h, int64_t src_stride_t,
                      const int32_t* jobs, int32_t n_jobs, void* stream);

/* Page source of one layer for lf_pack_pages_multi: element strides, channel stride 1. */
typedef struct lf_pack_source {
    const void* k;
    const void* v;
    int64_t stride_b, stride_h, stride_t;
} lf_pack_source;

/*
 * Page compress of several layers in one launch.  The reference flushes each
 * layer's full page inside that layer's commit (src/logitfill/packed/cache.py:
 * 48-81, one quantize_key_page + quantize_value_page per layer); every layer
 * of a decode step fills its page on the same token, so a caller that defers
 * the flushes to the end of the step packs all of them here at once (the
 * packed pages are read only by the next step).  Same results as one
 * lf_pack_pages call per layer.
 *
 * ``layers_host`` / ``srcs_host`` [n_layers]: host copies, used for the checks
 * and launch sizing; ``layers_dev`` / ``srcs_dev``: the same arrays in DEVICE
 * memory, read by the kernel.  ``jobs`` is a DEVICE int32 array [n_jobs][4] of
 * (layer, b, src_token0, dst_page).  Every layer must have the same n_kv and
 * take the fast shape (head_dim = page_size = k_group = v_group = 128,
 * bit_v 2, 16-byte aligned rows of a 2-byte dtype, even cap_tokens, 4-byte
 * aligned v_scale / v_min, 8-byte aligned v_code); otherwise LF_E_UNSUPPORTED
 * and nothing runs.  At most 2^21 jobs per call, else LF_E_SHAPE.
 */
int32_t lf_pack_pages_multi(const lf_packed_layer* layers_dev, const lf_packed_layer* layers_host,
                            const lf_pack_source* srcs_dev, const lf_pack_source* srcs_host, int32_t n_layers,
                            int32_t src_dtype, const int32_t* jobs, int32_t n_jobs, void* stream);

/*
 * Decode work plan (host function, no device access).  Sequence b's work is
 * its residual -- the BF16 tail page plus the new token, costed as
 * ``residual_pages`` pages -- and its ``hist_pages[b]`` packed pages.  It is
 * cut into ceil((hist_pages[b] + residual_pages) / pages_per_split) items of
 * equal work, (b, page_begin, page_end, kind): the first item (kind 2, or 1
 * when it holds no page) covers the residual and the pages left in its share,
 * the others (kind 0) pages only.  Writes ``work_out`` [n][4] and
 * ``seq_work_out`` [batch][2] = (first item, item count) of each sequence;
 * a sequence's items are consecutive.  Returns the item count n, or a
 * negative LF_E_* when ``work_cap`` is too small.  Both arrays must be copied
 * to the device before lf_decode_attention.  Any work list of this form is
 * valid input (sequences in any order, items of any sizes, several calls'
 * lists concatenated with b and the first items shifted): the matrix-core
 * kernel dispatches it in list order (workgroup item * n_kv + h), which the
 * Python layer uses to put larger items first.  An item's partial goes to the
 * workspace slot of its list position, or, when kind's bits 8..30 hold a value
 * s in 1 .. n_work, to slot s - 1: a list may then give the items in any
 * dispatch order while seq_work names each sequence's consecutive slots (the
 * Python layer's paired plan for a batch of equal sequences, where the
 * workgroups dispatched first, one per CU, take the larger items).
 */
int32_t lf_plan_decode(const int32_t* hist_pages, int32_t batch, int32_t pages_per_split, int32_t residual_pages,
                       int32_t* work_out, int32_t work_cap, int32_t* seq_work_out);

/* Decode-attention call arguments (see lf_decode_attention). */
typedef struct lf_decode_args {
    const void* query;  int32_t q_dtype;      /* [batch][n_q][head_dim]                 */
    const void* k_new;  const void* v_new;    /* [batch][n_kv][head_dim] or both NULL   */
    int32_t new_dtype;
    const void* tail_k; const void* tail_v;   /* [batch][n_kv][tail_cap][head_dim]      */
    int32_t tail_dtype, tail_cap;             /* 0 <= tail_cap <= page_size              */
    const int32_t* tail_len;                  /* device int32 [batch], each in
                                                 0 .. min(tail_cap, page_size - 1): a full
                                                 residual page must be packed (flushed)
                                                 first; both kernels clamp larger values
                                                 to that bound (a tail_len of page_size
                                                 leaves the page's last row out)           */
    void* out; int32_t out_dtype;             /* [batch][n_q][head_dim]                 */
    int32_t n_q;
    float scaling;                            /* softmax scale (reference: attn.scaling) */
    const int32_t* work;  int32_t n_work;     /* device, from lf_plan_decode            */
    const int32_t* seq_work;                  /* device, from lf_plan_decode            */
    void* workspace; int64_t workspace_bytes; /* >= lf_decode_workspace_bytes(); needs
                                                 no initialisation                      */
    int32_t kernel;                           /* 0 auto, 1 VALU, 2 MFMA                 */
    int32_t q_len;                            /* new query tokens per sequence (0 or 1:
                                                 one); with q_len > 1 the query and out are
                                                 [batch][n_q][q_len][head_dim], k_new/v_new
                                                 [batch][n_kv][q_len][head_dim], and the
                                                 workspace is sized for n_q * q_len rows  */
    const int32_t* work_host;                 /* optional (NULL): host copies of work and  */
    const int32_t* seq_work_host;             /* seq_work, the same values; a plan of at
                                                 most LF_INLINE_WORK items (LF_INLINE_SEQ
                                                 sequences) then travels in the kernels'
                                                 argument blocks, which saves each workgroup
                                                 a dependent read of device memory; read
                                                 during the call only                    */
    int32_t commit_new;                       /* 1: also append k_new / v_new (q_len rows)
                                                 to the tail at tail_len[b] and advance
                                                 tail_len, as lf_append_token would after
                                                 the call; needs tail buffers and, for every
                                                 sequence, tail_len + q_len < page_size (a
                                                 row past tail_cap is not written)        */
} lf_decode_args;

/* Plan sizes that travel inline in the kernel arguments when the host copies are given. */
#define LF_INLINE_WORK 208
#define LF_INLINE_SEQ 128

/* Workspace bytes for lf_decode_attention with ``n_work`` items: the fp32
 * partials [n_work][n_q][head_dim + 2] of the split-K items. */
int64_t lf_decode_workspace_bytes(int32_t n_q, int32_t head_dim, int32_t n_work);

/*
 * Decode attention for the new query token(s) of each sequence.  Replaces
 * logitfill_decode (reference src/logitfill/packed/kernel.cu:112-280) and the
 * dense fallback it protects (src/logitfill/packed/reference.py:30-56):
 *
 *   out[b, i] = softmax(scaling * q[b,i] . K_b^T) V_b,
 *   K_b = [dequant(history_b) ; tail_k[b, :, :tail_len[b]] ; k_new[b]]  (V likewise),
 *
 * with q head i reading kv head i / (n_q / n_kv).  With q_len > 1 new tokens (chunked
 * scoring / speculative decoding; reference reference.py:18-27,48), query token j sees the
 * whole history and tail and the new tokens 0..j (right-aligned causal mask); the (head,
 * token) pairs are served as n_q * q_len query rows, in tiles of rows across workgroups (any
 * number of rows per kv head).  Split-K over packed pages, then a second kernel merges the
 * splits' softmax partials; accumulation in fp32; output rounded to ``out_dtype``.  Requires
 * bit_v == 2 (as the reference kernel, reference.py:62), n_q % n_kv == 0, head_dim a power of
 * two in 8 .. 1024 (as kernel.cu:224-230) and at most 64 Value groups; other shapes return
 * LF_E_UNSUPPORTED (the Python layer then runs the dense dequantise-then-attend path on the
 * device, as the reference falls back to its dense path, reference.py:105-108).  ``kernel``
 * 0 takes the matrix-core kernel where its layout applies (head_dim 128, pages and Key groups
 * of 128 tokens, one Value group per row, some integer Key tier, the page-major Key scale/min
 * copy present, 16-byte aligned rows) and the general VALU kernel otherwise.
 */
int32_t lf_decode_attention(const lf_packed_layer* layer, const lf_decode_args* args, void* stream);

/*
 * Decode attention that allocates nothing (no counterpart in the reference): for callers
 * that cannot allocate device memory -- code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  Same arguments, checks, kernels and results as
 * lf_decode_attention, except that the split-K partials go to a file-scope device array of
 * LF_NOALLOC_SCRATCH_BYTES per GPU (held from library load until the process ends) and the
 * args' workspace / workspace_bytes are ignored.  A call whose partials
 * (lf_decode_workspace_bytes(n_q * q_len, head_dim, n_work)) exceed that size returns
 * LF_E_WORKSPACE and enqueues nothing.  The current HIP device must be the device of
 * ``stream`` and of every buffer.  All calls on one GPU share its array, and it keeps the
 * last call's partials: calls that overlap on one GPU (other streams or host threads) race.
 */
#define LF_NOALLOC_SCRATCH_BYTES (16u << 20)
int32_t lf_decode_attention_noalloc(const lf_packed_layer* layer, const lf_decode_args* args, void* stream);
int64_t lf_noalloc_scratch_bytes(void);

/*
 * Dense fp32 dequantisation of sequence b's first ``tokens`` history tokens
 * (reference src/logitfill/packed/layout.py:132-182, cache.py:83-90):
 * k_out, v_out fp32 [n_kv][tokens][head_dim], contiguous.
 */
int32_t lf_dequantize(const lf_packed_layer* layer, int32_t b, int32_t tokens,
                      float* k_out, float* v_out, void* stream);

/*
 * BF16 dense decode attention (comparator; no reference counterpart): the
 * same split-K/merge over bf16 K/V [batch][n_kv][tokens][head_dim] (element
 * strides kv_stride_b/h/t, multiples of 8; channel stride 1), query bf16
 * [batch][n_q][head_dim], out bf16, 16-byte aligned.  head_dim 128,
 * n_q / n_kv <= 8, tokens_per_split a multiple of 128 (LF_E_UNSUPPORTED /
 * LF_E_SHAPE otherwise).  Workspace as lf_dense_decode_workspace_bytes()
 * (fp32 partials, no initialisation).
 */
int64_t lf_dense_decode_workspace_bytes(int32_t batch, int32_t n_kv, int32_t n_q, int32_t head_dim,
                                        int32_t tokens, int32_t tokens_per_split);
int32_t lf_dense_decode(const void* query, const void* k, const void* v,
                        int32_t batch, int32_t n_q, int32_t n_kv, int32_t head_dim, int32_t tokens,
                        int64_t kv_stride_b, int64_t kv_stride_h, int64_t kv_stride_t,
                        float scaling, void* out, int32_t tokens_per_split,
                        void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Single-token append to the residual pages (the one-token commit of a decode step;
 * reference src/logitfill/packed/cache.py:48-62 while the page is not full).  For every
 * sequence b: the new Key and Value rows k_new / v_new [batch][n_kv][head_dim] (dtype
 * ``new_dtype``) are written, converted to ``tail_dtype``, as row tail_len[b] of tail_k / tail_v
 * [batch][n_kv][tail_cap][head_dim], and the DEVICE int32 tail_len[b] is advanced by one.  A
 * sequence whose residual page is already full (tail_len[b] >= tail_cap) is left unchanged:
 * full pages are packed (lf_pack_pages) and their length reset before the next append.  The
 * write position never leaves the device, so a decode step that appends needs no host copy.
 */
int32_t lf_append_token(void* tail_k, void* tail_v, int32_t tail_dtype, int32_t tail_cap, int32_t* tail_len,
                        const void* k_new, const void* v_new, int32_t new_dtype, int32_t batch, int32_t n_kv,
                        int32_t head_dim, void* stream);

/*
 * Layout helpers on the device (building blocks of the page packers, for callers of the
 * reference's layout module).  All arrays are contiguous device memory.
 *
 * lf_asymmetric_codes -- reference src/logitfill/packed/layout.py:12-18.  ``x`` holds
 * ``n_groups`` groups of ``group`` consecutive elements (dtype LF_BF16 / LF_FP16 /
 * LF_FP32, upcast to float32 exactly); per group lo = min, hi = max,
 * s = clamp((hi - lo) / (2^bits - 1), 1e-5, 1e5), code = clamp(rint((x - lo) / s), 0,
 * 2^bits - 1), all IEEE float32 (the reference's arithmetic on float32 tensors).
 * Writes codes int32 [n_groups][group], scale and lo float32 [n_groups].  1 <= bits <= 16.
 *
 * lf_pack_ints -- layout.py:21-35: LSB-first packing of each row of ``codes`` int32
 * [rows][n] (non-negative) into words int32 [rows][ceil(n / (32 / bits))]: slot j goes to
 * word j / per at bit (j % per) * bits, per = 32 / bits, missing slots are zero.
 *
 * lf_unpack_ints -- layout.py:38-46: the first ``count`` slots of each row of ``words``
 * int32 [rows][n_words] as codes int32 [rows][count]; count <= n_words * (32 / bits).
 *
 * 1 <= bits <= 32 for pack / unpack, as the reference's per = 32 // bits: a width that does
 * not divide 32 leaves the top 32 % bits bits of each word zero (3 bits: ten slots a word), a
 * width above 16 takes one slot a word (bits 32: the words themselves).
 */
int32_t lf_asymmetric_codes(const void* x, int32_t dtype, int64_t n_groups, int32_t group, int32_t bits,
                            int32_t* codes, float* scale, float* lo, void* stream);
int32_t lf_pack_ints(const int32_t* codes, int64_t rows, int32_t n, int32_t bits, int32_t* words, void* stream);
int32_t lf_unpack_ints(const int32_t* words, int64_t rows, int32_t n_words, int32_t count, int32_t bits,
                       int32_t* codes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOGITFILL_AMD_H */
