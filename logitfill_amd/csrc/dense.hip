// BF16 dense split-K decode attention on the gfx950 matrix cores: the comparator for the packed
// path (no reference counterpart; the reference's dense path is fp32 SDPA over dequantised
// history, src/logitfill/packed/reference.py:30-56).
//
// K/V bf16 [batch][n_kv][tokens][128] with element strides (b, h, t); query and output bf16
// [batch][n_q][128]; g = n_q / n_kv <= 8.  One workgroup of 4 waves per (split, batch, kv
// head) walks its split in pages of 128 tokens; wave w owns tokens 32w..32w+31 of each page
// (two 16-token MFMA tiles).
//
//   scores  S^T = K . Qb^T on v_mfma_f32_16x16x32_bf16: the A operand (lane: token row n16,
//           channels 32*kb + 8*s .. +7 for K-step s) comes straight from global memory as four
//           16-byte loads per tile, one page ahead; Qb holds q * scaling * log2(e) split into
//           bf16 hi (columns 0..7) and lo (columns 8..15), so one DPP add recombines them.
//   values  O = P' . V with P' = 2^(s - m) split hi (rows 0..7) / lo (rows 8..15): the score
//           accumulator layout is the A-operand layout, so probabilities feed the second MFMA in
//           place.  V pages arrive by LDS-DMA one page ahead (row-major, 16-byte chunks XOR-
//           swizzled by row); each lane takes its 8 tokens of one channel with two transpose
//           reads (ds_read_b64_tr_b16).
//
// Partials (o, m, l) per (split, head) go to the workspace; decode_reduce_kernel merges them.
#include "decode_common.hpp"

namespace lf {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kD = 128;
constexpr int kPageTok = 128;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kVTile = kPageTok * kD * 2;         // bytes of one V page in LDS
constexpr int kLds = 2 * kVTile + 1024;           // V ring of two + small
constexpr float kLazy = 8.f;                      // log2-domain headroom before the max moves

struct DenseParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    int64_t sb, sh, st;  // K/V element strides
    int n_q, n_kv, g, tokens, tps, n_splits;
    float qscale;
    float* part;         // [B * n_splits][n_kv][g][D + 2]
};

__device__ __forceinline__ float bf16f(uint16_t x) { return __uint_as_float(static_cast<uint32_t>(x) << 16); }

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const lds_void*)p)));
}
// The V rows stream through once: their DMA carries the non-temporal hint, as the packed kernel's
// pages do (208.7 -> 188.4 us per c2 layer-step in a same-box A/B).  The same hint on the K loads,
// which go straight into registers, made the kernel slower (209 -> 257 us), so they have none.
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds) : "memory");
}

// Max of x over the four 16-lane rows (permlane swaps; see decode_mfma.hip for why both
// swapped registers pass through an empty asm).
template <bool Half32>
__device__ __forceinline__ float swap_max(float x) {
    const int xi = __builtin_bit_cast(int, x);
    const auto r = Half32 ? __builtin_amdgcn_permlane32_swap(xi, xi, false, false)
                          : __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
    int r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
template <bool Half32>
__device__ __forceinline__ float swap_sum(float x) {
    const int xi = __builtin_bit_cast(int, x);
    const auto r = Half32 ? __builtin_amdgcn_permlane32_swap(xi, xi, false, false)
                          : __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
    int r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__global__ __launch_bounds__(kThreads, 2) void dense_decode_kernel(DenseParams p) {
    const int split = blockIdx.x;
    const int b = blockIdx.y / p.n_kv, h = blockIdx.y % p.n_kv;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, kb = lane >> 4;
    const int g = p.g;
    const int t0 = split * p.tps;
    const int t1 = min(p.tokens, t0 + p.tps);
    const int pages = (t1 - t0 + kPageTok - 1) / kPageTok;

    extern __shared__ __align__(16) unsigned char smem[];
    unsigned char* vring = smem;
    float* small = reinterpret_cast<float*>(smem + 2 * kVTile);
    float* alpha_lds = small;           // [waves][8]
    float* wstat = small + kWaves * 8;  // [waves][2][8]: m, l
    float* red = reinterpret_cast<float*>(smem);  // [waves][8][128], aliases the V ring after the loop

    const int64_t kvbase = static_cast<int64_t>(b) * p.sb + static_cast<int64_t>(h) * p.sh;

    // ---- Qb: B operand of K-step s, lane (n16, kb): q[head n16 % 8][32 kb + 8 s + j], hi or lo ----
    bf16x8 bq[4];
    {
        const int head = n16 & 7;
        const bool lo = n16 >= 8;
        const uint16_t* qrow = p.q + (static_cast<int64_t>(b) * p.n_q + h * g + head) * kD + 32 * kb;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            uint4 raw = {0, 0, 0, 0};
            if (head < g) raw = *reinterpret_cast<const uint4*>(qrow + 8 * s);
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = bf16f(static_cast<uint16_t>(w[j >> 1] >> (16 * (j & 1)))) * p.qscale;
                const __bf16 hi = static_cast<__bf16>(x);
                bq[s][j] = lo ? static_cast<__bf16>(x - static_cast<float>(hi)) : hi;
            }
        }
    }

    // ---- per-lane sources: K rows of the lane's two tiles, V chunks of the wave's DMA share ----
    const uint16_t* kp[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) kp[t] = p.k + kvbase + 32 * kb;
    const uint32_t ring = lds_addr(vring);
    // V DMA instruction i of wave w: block j = 4 i + w = tokens 4 j .. 4 j + 3, 16 chunks each.
    // Row r's 16-byte chunk k lands at chunk position k ^ 2 (r % 8): the transpose reads of the
    // value product (rows r0 .. r0 + 7 of one column pair per half wave) then hit 64 distinct
    // banks.
    auto v_dma = [&](int page, int slot) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int j = 4 * i + wave;
            const int row = 4 * j + (lane >> 4);
            const int tok = min(t0 + page * kPageTok + row, t1 - 1);
            const int chunk = (lane & 15) ^ (2 * (row & 7));
            dma16(p.v + kvbase + static_cast<int64_t>(tok) * p.st + 8 * chunk, ring + slot * kVTile + 1024 * j);
        }
    };
    auto k_load = [&](int page, uint4 (&kr)[2][4]) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int tok = min(t0 + page * kPageTok + 32 * wave + 16 * t + n16, t1 - 1);
            const uint4* src = reinterpret_cast<const uint4*>(kp[t] + static_cast<int64_t>(tok) * p.st);
#pragma unroll
            for (int s = 0; s < 4; ++s) kr[t][s] = src[s];
        }
    };

    float O[8][4];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[nt][r] = 0.f;
    float m_run = -__builtin_inff(), l_run = 0.f;

    uint4 kcur[2][4], knext[2][4];
    if (pages > 0) {
        v_dma(0, 0);
        k_load(0, kcur);
    }
    for (int page = 0; page < pages; ++page) {
        // V(page) and K(page) landed; every wave is done with page - 1 (its V slot is free).  The
        // wait is the builtin, not inline asm, so the compiler knows K(page) is in registers and
        // adds no wait of its own before the score products (which, with the V DMA of page + 1
        // ahead of it in the counter, would hold the scores until that page had landed too).
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) expcnt(7) lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (page + 1 < pages) {
            v_dma(page + 1, (page + 1) & 1);
            k_load(page + 1, knext);
        }
        // ---- scores of the wave's two tiles ----
        float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kcur[0][s]), bq[s], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kcur[1][s]), bq[s], acc1, 0, 0, 0);
        }
        // hi + lo columns; tokens past the split end score -inf
        const int tb = t0 + page * kPageTok + 32 * wave + 4 * kb;
        const float accs[8] = {acc0[0], acc0[1], acc0[2], acc0[3], acc1[0], acc1[1], acc1[2], acc1[3]};
        float sv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int xi = __builtin_bit_cast(int, accs[r]);
            const float sum = accs[r] + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x108, 0xf, 0xf, true));
            sv[r] = tb + (r & 3) + 16 * (r >> 2) < t1 ? sum : -__builtin_inff();
        }
        float mx = sv[0];
#pragma unroll
        for (int i = 1; i < 8; ++i) mx = fmaxf(mx, sv[i]);
        mx = swap_max<true>(swap_max<false>(mx));
        const bool grow = mx > m_run + kLazy;
        const float m_new = grow ? mx : m_run;
        const float m_off = m_new == -__builtin_inff() ? 0.f : m_new;
        float pp[8], psum = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pp[i] = __builtin_amdgcn_exp2f(sv[i] - m_off);
            psum += pp[i];
        }
        // A operand: k = 8 kb + j <-> token 4 kb + j (tile 0, j < 4) / 16 + 4 kb + j - 4 (tile 1);
        // hi in lanes n16 < 8, lo (moved 8 lanes up) in lanes n16 >= 8
        uint32_t ahi[4], alo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float x0 = pp[2 * j], x1 = pp[2 * j + 1];
            const __bf16 h0 = static_cast<__bf16>(x0), h1 = static_cast<__bf16>(x1);
            const __bf16 l0 = static_cast<__bf16>(x0 - static_cast<float>(h0));
            const __bf16 l1 = static_cast<__bf16>(x1 - static_cast<float>(h1));
            ahi[j] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h0)) | (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h1)) << 16);
            alo[j] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l0)) | (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, l1)) << 16);
        }
        uint4 au;
        au.x = __builtin_amdgcn_update_dpp(ahi[0], alo[0], 0x118, 0xf, 0xc, false);
        au.y = __builtin_amdgcn_update_dpp(ahi[1], alo[1], 0x118, 0xf, 0xc, false);
        au.z = __builtin_amdgcn_update_dpp(ahi[2], alo[2], 0x118, 0xf, 0xc, false);
        au.w = __builtin_amdgcn_update_dpp(ahi[3], alo[3], 0x118, 0xf, 0xc, false);
        const bf16x8 ap = __builtin_bit_cast(bf16x8, au);
        if (__builtin_amdgcn_ballot_w64(n16 < 8 && grow)) {
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
            if (kb == 0 && n16 < 8) alpha_lds[wave * 8 + n16] = alpha;
            __builtin_amdgcn_wave_barrier();
            const float4 arow = *reinterpret_cast<const float4*>(alpha_lds + wave * 8 + 4 * (kb & 1));
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                O[nt][0] *= arow.x;
                O[nt][1] *= arow.y;
                O[nt][2] *= arow.z;
                O[nt][3] *= arow.w;
            }
        }
        m_run = m_new;
        l_run += psum;
        // ---- values: B operand lane (n16, kb) = V[token of k][16 nt + n16] from the LDS page,
        // tokens r0 .. r0 + 3 and r0 + 16 .. r0 + 19 (r0 = 32 wave + 4 kb): two transpose reads
        // (ds_read_b64_tr_b16: lane i of a 16-lane group passes row i / 4, columns 4 (i % 4) ..
        // + 3 of a 4 x 16 block and receives column i) ----
        unsigned char* vt = vring + (page & 1) * kVTile;
        const int rr = 32 * wave + 4 * kb + (n16 >> 2);
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
            const int ch = 2 * nt + ((n16 >> 1) & 1);
            const int ra = rr, rb = rr + 16;
            typedef short v4i16 __attribute__((ext_vector_type(4)));
            const v4i16 ta = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<__attribute__((address_space(3))) v4i16*>(
                (lds_void*)(vt + ra * (kD * 2) + 16 * (ch ^ (2 * (ra & 7))) + 8 * (n16 & 1))));
            const v4i16 tb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<__attribute__((address_space(3))) v4i16*>(
                (lds_void*)(vt + rb * (kD * 2) + 16 * (ch ^ (2 * (rb & 7))) + 8 * (n16 & 1))));
            const uint2 ua = __builtin_bit_cast(uint2, ta), ub = __builtin_bit_cast(uint2, tb);
            const uint4 bu = {ua.x, ua.y, ub.x, ub.y};
            float4v o4 = {O[nt][0], O[nt][1], O[nt][2], O[nt][3]};
            o4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ap, __builtin_bit_cast(bf16x8, bu), o4, 0, 0, 0);
            O[nt][0] = o4[0]; O[nt][1] = o4[1]; O[nt][2] = o4[2]; O[nt][3] = o4[3];
        }
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int s = 0; s < 4; ++s) kcur[t][s] = knext[t][s];
    }
    // ---- merge: l over the lane groups, O rows r (hi) + r + 8 (lo), then the 4 waves ----
    l_run = swap_sum<true>(swap_sum<false>(l_run));
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[nt][r] = swap_sum<true>(O[nt][r]);
    __syncthreads();  // the V ring (aliased by red) is free
    if (kb < 2) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(wave * 8 + 4 * kb + r) * kD + 16 * nt + n16] = O[nt][r];
    }
    if (kb == 0 && n16 < 8) {
        wstat[(wave * 2 + 0) * 8 + n16] = m_run;
        wstat[(wave * 2 + 1) * 8 + n16] = l_run;
    }
    __syncthreads();
    const int item = b * p.n_splits + split;
    for (int e = tid; e < g * kD; e += kThreads) {
        const int i = e / kD, c = e % kD;
        float M = -__builtin_inff();
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, wstat[(w * 2 + 0) * 8 + i]);
        float o = 0.f, l = 0.f;
        if (M != -__builtin_inff()) {
            for (int w = 0; w < kWaves; ++w) {
                const float sc = __builtin_amdgcn_exp2f(wstat[(w * 2 + 0) * 8 + i] - M);
                o += sc * red[(w * 8 + i) * kD + c];
                l += sc * wstat[(w * 2 + 1) * 8 + i];
            }
        }
        float* rec = p.part + ((static_cast<int64_t>(item) * p.n_kv + h) * g + i) * (kD + 2);
        rec[c] = o;
        if (c == 0) {
            rec[kD] = M;
            rec[kD + 1] = l;
        }
    }
}

}  // namespace

int64_t dense_workspace_bytes(int batch, int n_kv, int n_q, int head_dim, int tokens, int tokens_per_split) {
    if (batch <= 0 || n_kv <= 0 || n_q <= 0 || head_dim <= 0 || tokens <= 0 || tokens_per_split <= 0) return LF_E_SHAPE;
    const int64_t splits = (tokens + tokens_per_split - 1) / tokens_per_split;
    return static_cast<int64_t>(batch) * splits * n_q * (head_dim + 2) * 4;
}

int launch_dense_decode(const void* query, const void* k, const void* v, int batch, int n_q, int n_kv, int head_dim,
                        int tokens, int64_t sb, int64_t sh, int64_t st, float scaling, void* out, int tps,
                        void* workspace, hipStream_t stream) {
    if (head_dim != kD) return LF_E_UNSUPPORTED;
    const int g = n_q / n_kv;
    if (g < 1 || g > 8) return LF_E_UNSUPPORTED;
    if (tps % kPageTok != 0) return LF_E_SHAPE;
    if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) | reinterpret_cast<uintptr_t>(query)) & 15)
        return LF_E_SHAPE;
    if ((st | sh | sb) & 7) return LF_E_SHAPE;  // rows must stay 16-byte aligned
    DenseParams p;
    p.q = static_cast<const uint16_t*>(query);
    p.k = static_cast<const uint16_t*>(k);
    p.v = static_cast<const uint16_t*>(v);
    p.sb = sb;
    p.sh = sh;
    p.st = st;
    p.n_q = n_q;
    p.n_kv = n_kv;
    p.g = g;
    p.tokens = tokens;
    p.tps = tps;
    p.n_splits = (tokens + tps - 1) / tps;
    p.qscale = scaling * 1.4426950408889634f;
    p.part = static_cast<float*>(workspace);
    const int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&dense_decode_kernel), kLds);
    if (rc != LF_OK) return rc;
    hipLaunchKernelGGL(dense_decode_kernel, dim3(p.n_splits, batch * n_kv), dim3(kThreads), kLds, stream, p);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return static_cast<int>(err);
    // merge the splits of each sequence with the packed path's reduce
    DecodeParams rp{};
    rp.L.head_dim = kD;
    rp.L.n_kv = n_kv;
    rp.L.batch = batch;
    rp.A.out = out;
    rp.A.out_dtype = LF_BF16;
    rp.A.n_q = n_q;
    rp.g = g;
    rp.part = p.part;
    rp.dense_splits = p.n_splits;
    return launch_decode_reduce(rp, stream);
}

}  // namespace lf
