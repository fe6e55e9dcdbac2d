// Packed decode attention, vector-ALU variant (fp32 FMA, one wave per work item).
//
// Reference: logitfill_decode_kernel, src/logitfill/packed/kernel.cu:112-190
// (dequantise Key through the tier map, int2 Value, online softmax), with the
// dense semantics of src/logitfill/packed/reference.py:30-56.  Differences in
// structure: one wave serves all g query heads of a kv head so the packed
// bytes are read once per kv head (the reference re-reads them per query head);
// the history is split across workgroups (split-K) and merged by decode_reduce_kernel.
//
// Per 64-token chunk a lane owns one token for the scores and one or more
// channels for the value accumulation.  The Key scale is folded into the
// query once per Key group:
//     score_i = sum_c q_ic (code_c s_c + m_c) = sum_slot (q s)_slot code_slot + sum_c q_ic m_c
// This kernel is the general path (any number of query rows per kv head, head_dim a power of two
// in 8..1024, up to 64 Value groups, Value rows of ceil(D / 16) words); the MFMA kernel covers
// the fast shapes.  Query rows are served in tiles of G rows (16, or 8 at head_dim 1024 to keep
// the LDS within 160 KB): workgroup (item, kv head, tile) holds rows G * tile .. + G - 1 of its kv
// head, so any GQA group (MQA included) and any number of new tokens stays on the kernel.
#include "decode_common.hpp"

namespace lf {
namespace {

// Query rows per workgroup (the row tile) at head_dim D.
__host__ __device__ constexpr int valu_tile_rows(int D) { return D > 512 ? 8 : 16; }

// Dynamic LDS of one workgroup (floats unless noted), in this order:
//   qT    [D][G]            q * scaling * log2(e), channel-major
//   p     [64][G]           probabilities of the current chunk
//   vsc   [64][v_groups]    Value scale per token and channel group
//   vmn   [64][v_groups]    Value min
//   vcode [64][v_words]     Value code words of the chunk (uint32)
//   qp    [n_slots][G]      q * Key scale per tier slot of the current Key group
struct ValuLds {
    int qT, p, vsc, vmn, vcode, qp, total;
};

__host__ __device__ inline ValuLds valu_lds(int D, int G, int v_groups, int v_words, int n_slots) {
    ValuLds o;
    int off = 0;
    o.qT = off;    off += D * G * 4;
    o.p = off;     off += 64 * G * 4;
    o.vsc = off;   off += 64 * v_groups * 4;
    o.vmn = off;   off += 64 * v_groups * 4;
    o.vcode = off; off += 64 * v_words * 4;
    o.qp = off;    off += n_slots * G * 4;
    o.total = off;
    return o;
}

__device__ __forceinline__ int slot_tier(const int* off, int slot) {
    return slot < off[1] ? 0 : slot < off[2] ? 1 : slot < off[3] ? 2 : 3;
}

template <int D>
__global__ __launch_bounds__(64) void decode_valu_kernel(DecodeParams p) {
    constexpr int kMaxG = valu_tile_rows(D);
    const lf_packed_layer& L = p.L;
    const lf_decode_args& A = p.A;
    const int item = blockIdx.x;
    const int h = blockIdx.y;
    const int lane = threadIdx.x;
    // rows row0 .. row0 + g - 1 of this kv head's p.g query rows (row = head * q_len + token)
    const int row0 = kMaxG * static_cast<int>(blockIdx.z);
    const int g = min(kMaxG, p.g - row0);
    const int* w4 = A.work + 4 * item;
    const int b = w4[0];
    const int pbeg = w4[1], pend = w4[2], kind = w4[3] & 0xff;
    // partial slot: kind bits 8.. hold slot + 1 for plans listed out of slot order
    const int part_slot = static_cast<unsigned>(w4[3] >> 8) - 1u < static_cast<unsigned>(A.n_work) ? (w4[3] >> 8) - 1 : item;

    int off[4];
    off[0] = 0;
    off[1] = L.k_width[0];
    off[2] = off[1] + L.k_width[1];
    off[3] = off[2] + L.k_width[2];
    const int n_slots = off[3] + L.k_width[3];
    const int vgs = L.v_groups;
    const int vws = L.v_words;
    const ValuLds lay = valu_lds(D, kMaxG, vgs, vws, n_slots);
    extern __shared__ __align__(16) unsigned char smem[];
    float* qT = reinterpret_cast<float*>(smem + lay.qT);        // [D][kMaxG]
    float* pb = reinterpret_cast<float*>(smem + lay.p);         // [64][kMaxG]
    float* vsc = reinterpret_cast<float*>(smem + lay.vsc);      // [64][vgs]
    float* vmn = reinterpret_cast<float*>(smem + lay.vmn);      // [64][vgs]
    uint32_t* vcode = reinterpret_cast<uint32_t*>(smem + lay.vcode);  // [64][vws]
    float* qp = reinterpret_cast<float*>(smem + lay.qp);        // [n_slots][kMaxG]

    // q, pre-scaled into the log2 domain.
    for (int idx = lane; idx < kMaxG * D; idx += 64) {
        const int i = idx / D, c = idx % D;
        float v = 0.f;
        if (i < g) v = load_as_f32(A.query, (static_cast<int64_t>(b) * A.n_q + h * p.g + row0 + i) * D + c, A.q_dtype);
        qT[c * kMaxG + i] = v * p.qscale;
    }
    __syncthreads();

    float m[kMaxG], lsum[kMaxG];
    constexpr int CPL = D >= 64 ? D / 64 : 1;  // channels per lane (lanes >= D idle when D < 64)
    float o[CPL][kMaxG];
#pragma unroll
    for (int i = 0; i < kMaxG; ++i) {
        m[i] = -__builtin_inff();
        lsum[i] = 0.f;
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc) o[cc][i] = 0.f;
    }

    // Online-softmax update with this lane's scores; publishes p into LDS.
    auto softmax_step = [&](float* score, bool active, float* alpha) {
#pragma unroll
        for (int i = 0; i < kMaxG; ++i) {
            if (i < g) {
                const float s = active ? score[i] : -__builtin_inff();
                const float mnew = fmaxf(m[i], wave_max(s));
                alpha[i] = mnew == -__builtin_inff() ? 1.f : __builtin_amdgcn_exp2f(m[i] - mnew);
                const float pi = active ? __builtin_amdgcn_exp2f(s - mnew) : 0.f;
                lsum[i] = lsum[i] * alpha[i] + pi;
                m[i] = mnew;
                pb[lane * kMaxG + i] = pi;
            }
        }
    };

    if (kind != 1) {  // pages (kind 0, 2)
        const int kg = L.k_group;
        const int chunk = kg < 64 ? kg : 64;
        const int64_t tok_end = static_cast<int64_t>(pend) * L.page_size;
        for (int64_t tok = static_cast<int64_t>(pbeg) * L.page_size; tok < tok_end; tok += kg) {
            const int64_t kgi = tok / kg;
            // Fold this Key group's scale into q; collect sum_c q_c m_c.
            float bias[kMaxG];
#pragma unroll
            for (int i = 0; i < kMaxG; ++i) bias[i] = 0.f;
            __syncthreads();
            for (int slot = lane; slot < n_slots; slot += 64) {
                const int t = slot_tier(off, slot);
                const int j = slot - off[t];
                const int cnt = L.tier_count[t][h];
                float* row = qp + slot * kMaxG;
                if (j >= cnt) {
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i) row[i] = 0.f;
                    continue;
                }
                const int c = L.tier_index[t][h * L.k_width[t] + j];
                if (t == 3) {
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i) row[i] = qT[c * kMaxG + i];
                } else {
                    const int64_t gi = kgrp_idx(L, b, h, L.k_width[t], j, kgi);
                    const float s = f16_to_f32(L.k_scale[t][gi]);
                    const float mn = f16_to_f32(L.k_min[t][gi]);
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i) {
                        row[i] = qT[c * kMaxG + i] * s;
                        bias[i] += qT[c * kMaxG + i] * mn;
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kMaxG; ++i) bias[i] = wave_sum(bias[i]);
            __syncthreads();
            // Process the group's chunks.
            for (int64_t t0 = tok; t0 < tok + kg; t0 += chunk) {
                const bool active = lane < chunk;
                const int64_t row = tok_row(L, b, h, t0 + (active ? lane : 0));
                float score[kMaxG];
#pragma unroll
                for (int i = 0; i < kMaxG; ++i) score[i] = bias[i];
                for (int t = 0; t < 3; ++t) {
                    const int words = L.k_words[t];
                    const int bits = 2 << t;
                    const int per = 32 / bits;
                    const uint32_t mask = (1u << bits) - 1u;
                    const int width = L.k_width[t];
                    for (int w = 0; w < words; ++w) {
                        const uint32_t word = static_cast<uint32_t>(L.k_code[t][row * words + w]);
                        const int kmax = min(per, width - w * per);
                        for (int k = 0; k < kmax; ++k) {
                            const float cf = static_cast<float>((word >> (k * bits)) & mask);
                            const float* qrow = qp + (off[t] + w * per + k) * kMaxG;
#pragma unroll
                            for (int i = 0; i < kMaxG; ++i)
                                if (i < g) score[i] = fmaf(qrow[i], cf, score[i]);
                        }
                    }
                }
                for (int j = 0; j < L.k_width[3]; ++j) {
                    const float v = f16_to_f32(L.k_value16[row * L.k_width[3] + j]);
                    const float* qrow = qp + (off[3] + j) * kMaxG;
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i)
                        if (i < g) score[i] = fmaf(qrow[i], v, score[i]);
                }
                float alpha[kMaxG];
                softmax_step(score, active, alpha);
                if (active) {
                    for (int vg = 0; vg < vgs; ++vg) {
                        vsc[lane * vgs + vg] = f16_to_f32(L.v_scale[row * vgs + vg]);
                        vmn[lane * vgs + vg] = f16_to_f32(L.v_min[row * vgs + vg]);
                    }
                    for (int w = 0; w < vws; ++w) vcode[lane * vws + w] = static_cast<uint32_t>(L.v_code[row * vws + w]);
                }
                __syncthreads();
#pragma unroll
                for (int cc = 0; cc < CPL; ++cc) {
                    const int c = lane + 64 * cc;
                    const int vg = (c < D ? c : 0) / L.v_group;
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i) o[cc][i] *= alpha[i];
                    if (c >= D) continue;
                    for (int tt = 0; tt < chunk; ++tt) {
                        const uint32_t code = (vcode[tt * vws + (c >> 4)] >> (2 * (c & 15))) & 3u;
                        const float v = static_cast<float>(code) * vsc[tt * vgs + vg] + vmn[tt * vgs + vg];
#pragma unroll
                        for (int i = 0; i < kMaxG; ++i)
                            if (i < g) o[cc][i] = fmaf(pb[tt * kMaxG + i], v, o[cc][i]);
                    }
                }
                __syncthreads();
            }
        }
    }
    if (kind != 0) {
        // Residual (kind 1, 2): the BF16 tail page then the new token(s) (reference.py:35-44).
        // With q_len new tokens, row i (token i % q_len) sees new tokens 0 .. i % q_len
        // (reference.py:18-27,48: the causal mask is right-aligned).  tail_len is clamped to
        // min(tail_cap, page_size - 1), as in the matrix-core kernel: a full residual page is
        // packed before decode reads it, and a tail_len of page_size leaves the last row out.
        const int tl = min(max(A.tail_len[b], 0), min(A.tail_cap, L.page_size - 1));
        const int q_len = p.q_len;
        const int n_new = A.k_new != nullptr ? q_len : 0;
        const int n_res = tl + n_new;
        const int64_t new_row0 = (static_cast<int64_t>(b) * L.n_kv + h) * q_len;  // first new row
        for (int t0 = 0; t0 < n_res; t0 += 64) {
            const int tt_lane = t0 + lane;
            const bool active = tt_lane < n_res;
            const void* kp;
            int64_t kbase;
            int kdt;
            if (tt_lane < tl) {
                kp = A.tail_k;
                kbase = ((static_cast<int64_t>(b) * L.n_kv + h) * A.tail_cap + tt_lane) * D;
                kdt = A.tail_dtype;
            } else {
                kp = A.k_new;
                kbase = (new_row0 + (active ? tt_lane - tl : 0)) * D;
                kdt = A.new_dtype;
            }
            float score[kMaxG];
#pragma unroll
            for (int i = 0; i < kMaxG; ++i) score[i] = 0.f;
            if (active) {
                for (int c = 0; c < D; ++c) {
                    const float k = load_as_f32(kp, kbase + c, kdt);
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i)
                        if (i < g) score[i] = fmaf(qT[c * kMaxG + i], k, score[i]);
                }
                if (tt_lane >= tl && q_len > 1) {
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i)
                        if (tt_lane - tl > (row0 + i) % q_len) score[i] = -__builtin_inff();
                }
            }
            float alpha[kMaxG];
            softmax_step(score, active, alpha);
            __syncthreads();
            const int cnt = min(64, n_res - t0);
#pragma unroll
            for (int cc = 0; cc < CPL; ++cc) {
                const int c = lane + 64 * cc;
#pragma unroll
                for (int i = 0; i < kMaxG; ++i) o[cc][i] *= alpha[i];
                if (c >= D) continue;
                for (int tt = 0; tt < cnt; ++tt) {
                    const int tok = t0 + tt;
                    float v;
                    if (tok < tl)
                        v = load_as_f32(A.tail_v, ((static_cast<int64_t>(b) * L.n_kv + h) * A.tail_cap + tok) * D + c,
                                        A.tail_dtype);
                    else
                        v = load_as_f32(A.v_new, (new_row0 + tok - tl) * D + c, A.new_dtype);
#pragma unroll
                    for (int i = 0; i < kMaxG; ++i)
                        if (i < g) o[cc][i] = fmaf(pb[tt * kMaxG + i], v, o[cc][i]);
                }
            }
            __syncthreads();
        }
    }

    // Partials: o per lane-channel, m uniform, l reduced across the wave.
    for (int i = 0; i < g; ++i) {
        float* r = part_rec(p, part_slot, h, row0 + i);
#pragma unroll
        for (int cc = 0; cc < CPL; ++cc)
            if (lane + 64 * cc < D) r[lane + 64 * cc] = o[cc][i];
        const float lt = wave_sum(lsum[i]);
        if (lane == 0) {
            r[D] = m[i];
            r[D + 1] = lt;
        }
    }
    if (A.commit_new && kind != 0 && blockIdx.z == 0) commit_new_rows(p, b, h, lane, 64);
}

template <int D>
int launch_valu_d(const DecodeParams& p, size_t lds, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(&decode_valu_kernel<D>);
    const int rc = allow_dynamic_lds(fn, lds);
    if (rc != LF_OK) return rc;
    const int tiles = (p.g + valu_tile_rows(D) - 1) / valu_tile_rows(D);
    hipLaunchKernelGGL(decode_valu_kernel<D>, dim3(p.A.n_work, p.L.n_kv, tiles), dim3(64), lds, stream, p);
    return LF_OK;
}

}  // namespace

int launch_decode_valu(const DecodeParams& p, hipStream_t stream) {
    const int D = p.L.head_dim;
    const int n_slots = p.L.k_width[0] + p.L.k_width[1] + p.L.k_width[2] + p.L.k_width[3];
    const size_t lds = static_cast<size_t>(valu_lds(D, valu_tile_rows(D), p.L.v_groups, p.L.v_words, n_slots).total);
    if (lds > 160 * 1024) return LF_E_UNSUPPORTED;
    if ((p.g + valu_tile_rows(D) - 1) / valu_tile_rows(D) > 65535) return LF_E_SHAPE;  // grid z
    int rc;
    switch (D) {
        case 8: rc = launch_valu_d<8>(p, lds, stream); break;
        case 16: rc = launch_valu_d<16>(p, lds, stream); break;
        case 32: rc = launch_valu_d<32>(p, lds, stream); break;
        case 64: rc = launch_valu_d<64>(p, lds, stream); break;
        case 128: rc = launch_valu_d<128>(p, lds, stream); break;
        case 256: rc = launch_valu_d<256>(p, lds, stream); break;
        case 512: rc = launch_valu_d<512>(p, lds, stream); break;
        case 1024: rc = launch_valu_d<1024>(p, lds, stream); break;
        default: return LF_E_UNSUPPORTED;
    }
    if (rc != LF_OK) return rc;
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return static_cast<int>(err);
    return launch_decode_reduce(p, stream);
}

}  // namespace lf
