// Packed decode attention on the gfx950 matrix cores (v_mfma_f32_16x16x32_f16).
//
// Reference semantics: src/logitfill/packed/reference.py:30-56 (dense dequantise,
// softmax attention over [history ; tail ; new]); replaces the CUDA kernel
// src/logitfill/packed/kernel.cu:112-190.  Shapes served: head_dim 128,
// page = Key group = 128 tokens, one Value group per token (v_group 128), int2
// Values, any number of query rows per kv head ((n_q / n_kv) * q_len, row = head * q_len +
// token, served 8 rows per workgroup).  Anything else runs the VALU kernel.
//
// Work: one workgroup of 4 waves per (split item, kv head, tile of 8 query rows); wave w computes
// tokens 32w..32w+31 (two 16-token tiles) of every page of the item.  Pages arrive by LDS-DMA
// (global_load_lds, 16-byte chunks: the Key codes, the Value scales / mins / codes, the fp16-tier
// rows and the page's block of the page-major Key scale/min copy k_sm_page) into a ring of two
// page slots, one page ahead of the page being computed.
// Per page: a barrier (the page landed, the previous page is computed), the page's
// "preparation" (the per-page operands below) into the one prepared buffer by all waves, a
// second barrier, then the compute.  Partials (m, l, o) of each item go to the workspace;
// decode_reduce_kernel merges them.  (A third slot, two pages in flight, measured no faster.)
//
// Scores.  With the Key scale folded into the query once per page,
//     s[t][i] = sum_slot Qs[i][slot] * code[t][slot] + sum_c q_ic * min_c,
//     Qs = q * scaling * log2(e) * scale_slot,
// computed as S^T = Codes . Qs^T: the K dimension is the page's slots ordered
// tier by tier in blocks of 8 codes; a K-step of 32 covers four blocks of one
// tier.  A code becomes the fp16 value beta + code by placing its bits in the
// mantissa under a fixed exponent (beta = 16 or 4 for int2, 256 or 16 for
// int4, 1024 for int8, no transform for the fp16 tier); sum_slot Qs * beta
// moves into the per-page bias.  Qs is split hi + lo in fp16 across columns
// 0..7 / 8..15 (the GQA group has at most 8 heads) and one DPP add
// recombines them.
//
// Values.  The S^T accumulator layout (lane: head n = lane%16, tokens 4*kb+r
// of each of the wave's two 16-token tiles, kb = lane/16) is the A-operand
// layout of O = P' . (4 + code_V) with k = those 8 tokens, so probabilities
// feed the second MFMA in place (4 + c from the same exponent-field unpack).
// P' = p * vscale is split hi/lo across rows 0..7 / 8..15; the constant
// vmin - 4 * vscale enters through sum_t p_t * mid_t.  Value codes are
// regrouped per page (one dword = one byte column of 4 consecutive tokens) so
// each lane's 8 codes for one 16-channel tile are two LDS dwords.
#include <type_traits>

#include <cstring>

#include "decode_common.hpp"

namespace lf {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 128;
constexpr int kPage = 128;
constexpr int kMaxDma = 8;    // 16-byte DMA instructions per wave per page (<= 2048 chunks)
constexpr int kMaxKSteps = 16; // K-steps of a page: at most 4 per tier (128 channels)
constexpr float kLazyRescale = 8.f;  // log2-domain headroom before the running max moves
constexpr int kRawbVs = 0;    // rest buffer: Value scale [128] fp16
constexpr int kRawbVm = 256;  //              Value min [128] fp16
constexpr int kRawbVc = 512;  //              Value codes [128][8] u32
constexpr int kRawbF16 = 4608;  //            fp16-tier rows [128][width16]
// Prepared buffer: fixed offsets first (they become immediate offsets of the LDS accesses).
constexpr int kCkVsc = 0;       // [128] fp32 Value scale
constexpr int kCkVmid = 512;    // [128] fp32 vmin - 4 * vscale
constexpr int kCkBias = 1024;   // [8 heads][4 waves] fp32 page bias partials
constexpr int kCkVt = 1152;     // [32 groups][36] u32 Value-code byte columns (4 per 8-word row) + 4 pad
constexpr int kCkQs = kCkVt + 32 * 36 * 4;  // [nb][16][8] fp16 Qs hi (rows 0..7) / lo (rows 8..15)
static_assert(kCkQs >= 8 * kD * 4, "the item prologue's q [8][128] fp32 lies below the fp16-tier Qs");

struct MfmaLayout {
    int kst[4];          // K-steps per tier (int2: even; K-step s takes half s&1 of 4 words)
    int kfirst[4];       // first K-step of each tier
    int nb;              // padded blocks (4 per K-step)
    int nb_int;          // padded blocks of the integer tiers (the page-major scale/min block's)
    int w16p;            // fp16-tier row stride in the prepared buffer (multiple of 8)
    int seg_end[3];      // cumulative 16-byte chunks of the Key-code rows K0, K1, K2 (region A)
    int n_chunks;        // region A + region B chunks
    int ja, jb;          // 64-chunk DMA blocks of the Key codes (chunks [0, seg_end[2])) and of the rest
    int rawa_bytes;      // Key-code buffer: K0, K1, K2 rows of the page, padded to whole DMA blocks
    int rawb_sm;         // rest buffer (v scale at 0, v min at 256, [128][8] u32 Value codes at 512,
                         // fp16-tier rows at 4608, padded to whole DMA blocks): the page's
                         // k_sm_page block [nb_int][8 scales, 8 mins] fp16 at this offset
    int rawb_bytes;
    int ck_v16;          // prepared: [128][w16p] fp16 Key fp16 tier, zero padded (after Qs), one spare dword
    int ck_bytes;
    int off_qperm;       // [nb][2][8 heads][4] fp32: q * scaling*log2e per slot (0 for padding), a block's
                         // positions 0..3 of the 8 heads, then its positions 4..7 (a 16-byte read
                         // per lane and half, consecutive lanes at consecutive addresses)
    int off_small;       // alpha [waves][8], wave m/l/mid [waves][3][8]
    int slot_bytes;      // one page slot: Key-code buffer, then rest buffer
    int off_ck;          // the prepared buffer
    int off_raw;         // two page slots (prepared buffer + page slots form one alias region)
    int lds_bytes;
};



// s_waitcnt vmcnt(n) lgkmcnt(0); s_barrier, for n in {0, 1, ..., 15} (larger n waits for
// everything): this wave's older DMA and all its LDS operations are done, newer DMA may still
// be in flight.  The asm memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void dma_barrier(int n) {
#define LF_W(N) case N: asm volatile("s_waitcnt vmcnt(" #N ") lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    switch (n) {
        LF_W(0) LF_W(1) LF_W(2) LF_W(3) LF_W(4) LF_W(5) LF_W(6) LF_W(7)
        LF_W(8) LF_W(9) LF_W(10) LF_W(11) LF_W(12) LF_W(13) LF_W(14) LF_W(15)
        default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    }
#undef LF_W
}

// s_waitcnt lgkmcnt(0); s_barrier: every wave's LDS operations are done; DMA in flight stays
// in flight (__syncthreads would also wait for it).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// a[t] for a run-time t in 0..3 (or 0..2) of a kernel-argument array, through selects over
// SGPR copies.  A dynamic index into the argument block would copy it to scratch memory; a plain
// select chain with a per-lane t the compiler turns into a select of *addresses* and one vector
// load from the argument block per lane -- a memory round trip each, in the prologue's
// dependent chain.  The empty asm pins the four values in SGPRs (scalar loads, already
// prefetched), so the select is four VALU ops.
template <class T>
__device__ __forceinline__ T sel4(const T (&a)[4], int t) {
    T a0 = a[0], a1 = a[1], a2 = a[2], a3 = a[3];
    asm volatile("" : "+s"(a0), "+s"(a1), "+s"(a2), "+s"(a3));
    return t == 0 ? a0 : t == 1 ? a1 : t == 2 ? a2 : a3;
}

// LDS-DMA: each lane's 16 bytes at ``g`` land at lds + 16 * lane.  Issued through asm so the
// compiler does not order every later LDS read behind it (it cannot tell the buffers apart and
// would wait for all DMA in flight); the waits are explicit instead.  The compiler writes M0 just
// before the asm; an LDS-DMA instruction needs one wait state after an SALU write of M0, hence
// the s_nop.  The load carries the non-temporal (streaming) cache hint: the L2 evicts those
// lines first and keeps what the launch reads again (its instructions, arguments, q) and the
// partials the reduce kernel reads next (c2: 71.7 -> 70.6 us per layer-step, c1 21.5 -> 20.9 in
// a same-box A/B; several row tiles of one kv head still find the pages in L2).
__device__ __forceinline__ uint32_t lds_addr(unsigned char* p) {
    return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)p)));
}
__device__ __forceinline__ void dma16(const unsigned char* g, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(lds) : "memory");
}

// Bit patterns of the exponent-field code unpack, held in VGPRs: with register operands the
// compiler selects (x & mask) | bits as one v_and_or_b32 (VOP3 takes no literal), and the
// unpack stays compiler-visible code, so the compiler also inserts the wait states an MFMA
// needs after a VALU write of its operands.  ``as_vgpr`` hides the constant from folding.
struct UnpackBits {
    uint32_t m2lo, m2hi;    // int2 code at mantissa bits 6..7 / 8..9 (both halves)
    uint32_t m4lo, m4hi;    // int4 code at mantissa bits 2..5 / 6..9
    uint32_t e16, e4, e256; // fp16 exponent fields of 16, 4, 256 (both halves)
};

__device__ __forceinline__ uint32_t as_vgpr(uint32_t s) {
    uint32_t v;
    asm("v_mov_b32 %0, %1" : "=v"(v) : "s"(s));
    return v;
}

__device__ __forceinline__ UnpackBits vgpr_bits(const UnpackBits& k) {
    return UnpackBits{as_vgpr(k.m2lo), as_vgpr(k.m2hi), as_vgpr(k.m4lo), as_vgpr(k.m4hi),
                      as_vgpr(k.e16),  as_vgpr(k.e4),   as_vgpr(k.e256)};
}

__device__ __forceinline__ uint32_t bfi(uint32_t x, uint32_t mask, uint32_t bits) { return (x & mask) | bits; }

struct MfmaParams {
    DecodeParams p;
    MfmaLayout y;
    UnpackBits k;
    int res_mfma;  // residual pass: 0 VALU, 1 bf16 matrix cores, 2 fp16 matrix cores (residual_mfma)
    int n_rt;      // row tiles per kv head: ceil(p.g / 8)
    int inline_work;  // 1: work_inline holds the plan (2-D grid, n_work <= LF_INLINE_WORK)
    int pad_[3];
    int32_t work_inline[4 * LF_INLINE_WORK];  // the work list, when inline_work
};
static_assert(sizeof(MfmaParams) <= 4096, "kernel arguments are limited to 4 KB");

// Tier-local ranks of positions 0..7 of local block ``lb``.  Register r of a block (positions
// 2r, 2r+1) holds the code pair the unpack helpers below produce: int2 -- word 4 (lb / 8) + lb % 4,
// half (lb / 4) % 2: codes (4 half + r, 4 half + r + 8); int4 word lb: codes (r, r + 4); int8 words
// 2 lb, 2 lb + 1: bytes (r & 1, + 2); fp16: natural order.  Computed for a per-lane tier without
// branches: a base per tier plus the position's offset, packed as 4-bit fields.
__device__ __forceinline__ void block_slots(int tier, int lb, int (&slot)[8]) {
    const int base = tier == 0 ? 16 * (4 * (lb >> 3) + (lb & 3)) + 4 * ((lb >> 2) & 1) : 8 * lb;
    const uint32_t offs = tier == 0 ? 0xB3A29180u : tier == 1 ? 0x73625140u : tier == 2 ? 0x75643120u : 0x76543210u;
#pragma unroll
    for (int pos = 0; pos < 8; ++pos) slot[pos] = base + static_cast<int>((offs >> (4 * pos)) & 15u);
}

// Is local block ``lb`` of ``tier`` backed by stored words?  (Selects, no branches.)
__device__ __forceinline__ bool block_live(const lf_packed_layer& L, int tier, int lb) {
    const int v = tier == 0 ? 4 * (lb >> 3) + (lb & 3) : tier == 1 ? lb : tier == 2 ? 2 * lb : 8 * lb;
    const int lims[4] = {L.k_words[0], L.k_words[1], L.k_words[2], L.k_width[3]};
    return v < sel4(lims, tier);
}

// int2, half H of word w: registers r = (code 4H+r, code 4H+r+8); even r: bits to mantissa
// 6..7 under exponent 16 (16 + c), odd r: bits 8..9 under exponent 4 (4 + c).
template <int H>
__device__ __forceinline__ half8 unpack2(uint32_t w, const UnpackBits& k) {
    const uint32_t y1 = H == 0 ? (w << 6) : (w >> 2);
    const uint32_t y2 = H == 0 ? (w << 2) : (w >> 6);
    const uint4 u = {bfi(y1, k.m2lo, k.e16), bfi(y1, k.m2hi, k.e4), bfi(y2, k.m2lo, k.e16), bfi(y2, k.m2hi, k.e4)};
    return __builtin_bit_cast(half8, u);
}

// int4 word: registers r = (code r, code r+4); even r: mantissa 2..5 under 256 (256 + c),
// odd r: mantissa 6..9 under 16 (16 + c).
__device__ __forceinline__ half8 unpack4(uint32_t w, const UnpackBits& k) {
    const uint32_t y1 = w << 2, y2 = w >> 6;
    const uint4 u = {bfi(y1, k.m4lo, k.e256), bfi(y1, k.m4hi, k.e16), bfi(y2, k.m4lo, k.e256), bfi(y2, k.m4hi, k.e16)};
    return __builtin_bit_cast(half8, u);
}

// int8 words w0, w1: registers (bytes 0, 2), (1, 3) of each under a 0x64 high byte (1024 + c).
__device__ __forceinline__ half8 unpack8(uint32_t w0, uint32_t w1) {
    const uint4 u = {__builtin_amdgcn_perm(w0, 0x64646464u, 0x00060004u), __builtin_amdgcn_perm(w0, 0x64646464u, 0x00070005u),
                     __builtin_amdgcn_perm(w1, 0x64646464u, 0x00060004u), __builtin_amdgcn_perm(w1, 0x64646464u, 0x00070005u)};
    return __builtin_bit_cast(half8, u);
}

// 4x4 byte transpose: out[k] = (a0.byte k, a1.byte k, a2.byte k, a3.byte k).
__device__ __forceinline__ void byte_transpose4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t* o) {
    const uint32_t t01_lo = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
    const uint32_t t01_hi = __builtin_amdgcn_perm(a1, a0, 0x07030602u);
    const uint32_t t23_lo = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
    const uint32_t t23_hi = __builtin_amdgcn_perm(a3, a2, 0x07030602u);
    o[0] = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(t23_lo, t01_lo, 0x07060302u);
    o[2] = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x05040100u);
    o[3] = __builtin_amdgcn_perm(t23_hi, t01_hi, 0x07060302u);
}

// Loop-invariant layout values, each in a scalar register of its own.  Read straight from the
// kernel argument, the compiler keeps 16 consecutive argument dwords as one register tuple and
// spills and reloads the tuple whole inside the page loop.
struct LoopY {
    int kst0, kst1, kst2, kst3, kf1, kf2, kf3, nb, nb_int, w16p;
    int seg0, seg1, ja, rawa_bytes, rawb_sm, slot_bytes, ck_v16;
};

__device__ __forceinline__ LoopY loop_y(const MfmaLayout& y) {
    LoopY z{y.kst[0], y.kst[1], y.kst[2], y.kst[3], y.kfirst[1], y.kfirst[2], y.kfirst[3], y.nb, y.nb_int, y.w16p,
            y.seg_end[0], y.seg_end[1], y.ja, y.rawa_bytes, y.rawb_sm, y.slot_bytes, y.ck_v16};
    asm volatile("" : "+s"(z.kst0), "+s"(z.kst1), "+s"(z.kst2), "+s"(z.kst3), "+s"(z.kf1), "+s"(z.kf2), "+s"(z.kf3),
                      "+s"(z.nb), "+s"(z.nb_int), "+s"(z.w16p));
    asm volatile("" : "+s"(z.seg0), "+s"(z.seg1), "+s"(z.ja), "+s"(z.rawa_bytes), "+s"(z.rawb_sm),
                      "+s"(z.slot_bytes), "+s"(z.ck_v16));
    return z;
}

// Operands of one Qs block: q of (block, head) and the block's 8 Key scales and 8 Key mins
// (fp16, from the page's k_sm_page block).
struct QsRegs {
    float4 q0, q1;
    uint4 s, m;
};

__device__ __forceinline__ void qs_fetch(const float* qrow, const unsigned char* smb, QsRegs& r) {
    r.q0 = *reinterpret_cast<const float4*>(qrow);
    r.q1 = *reinterpret_cast<const float4*>(qrow + 32);
    r.s = *reinterpret_cast<const uint4*>(smb);
    r.m = *reinterpret_cast<const uint4*>(smb + 16);
}

// Qs of an integer-tier block for one head -- hi into ``qs_hi``, lo (the fp16 residual) into
// ``qs_lo`` -- and the block's share of the bias sum_slot q * (min - beta * scale).  Padding
// slots have q == 0 and scale 1.0, min 0.0.  Written so the compiler uses mixed-precision FMAs
// on the fp16 halves directly.
__device__ __forceinline__ float qs_math(const QsRegs& r, half8* qs_hi, half8* qs_lo, float beta_lo, float beta_hi) {
    const float qv[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
    const uint32_t sw[4] = {r.s.x, r.s.y, r.s.z, r.s.w};
    const uint32_t mw[4] = {r.m.x, r.m.y, r.m.z, r.m.w};
    half8 hi, lo;
    float bsum = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const _Float16 sc = __builtin_bit_cast(half2v, sw[k >> 1])[k & 1];
        const _Float16 mn = __builtin_bit_cast(half2v, mw[k >> 1])[k & 1];
        const _Float16 hk = static_cast<_Float16>(fmaf(qv[k], static_cast<float>(sc), 0.f));
        hi[k] = hk;
        lo[k] = static_cast<_Float16>(fmaf(qv[k], static_cast<float>(sc), -static_cast<float>(hk)));
        // positions with (k & 2) == 0 unpack under beta_lo, the others under beta_hi
        const float mp = fmaf((k & 2) ? -beta_hi : -beta_lo, static_cast<float>(sc), static_cast<float>(mn));
        bsum = fmaf(qv[k], mp, bsum);
    }
    *qs_hi = hi;
    *qs_lo = lo;
    return bsum;
}

// Max / sum of x over the four 16-lane rows (lanes l, l ^ 16, l ^ 32, l ^ 48), in every lane:
// v_permlane16_swap pairs rows (0, 1), (2, 3); v_permlane32_swap pairs the wave halves.  Both
// swapped registers pass through an empty asm: this compiler otherwise takes the two results
// of a swap to be equal and drops the second.
template <bool Half32>
__device__ __forceinline__ void swap_rows(float x, float& a, float& b) {
    const int xi = __builtin_bit_cast(int, x);
    const auto r = Half32 ? __builtin_amdgcn_permlane32_swap(xi, xi, false, false)
                          : __builtin_amdgcn_permlane16_swap(xi, xi, false, false);
    int r0 = r[0], r1 = r[1];
    asm volatile("" : "+v"(r0), "+v"(r1));
    a = __builtin_bit_cast(float, r0);
    b = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float halves_sum(float x) {
    float a, b;
    swap_rows<true>(x, a, b);
    return a + b;
}
__device__ __forceinline__ float rows_sum(float x) {
    float a, b;
    swap_rows<false>(x, a, b);
    return halves_sum(a + b);
}
__device__ __forceinline__ float rows_max(float x) {
    float a, b;
    swap_rows<false>(x, a, b);
    swap_rows<true>(fmaxf(a, b), a, b);
    return fmaxf(a, b);
}

// Per-lane DMA state.  A page is fetched as 16-byte chunks in two regions -- region A: the
// Key-code rows K0, K1, K2; region B: Value scale, Value min, Value codes, fp16-tier rows and the
// page's k_sm_page block.  Block j (64 chunks) of region A lands in the Key-code buffer at 1024 j,
// block j of region B in the rest buffer at 1024 j.  Wave w issues blocks w, w + 4, ...  Every
// lane of an issued instruction loads: lanes past a region's last chunk re-read that chunk into
// the block padding of their buffer.
struct DmaSrc {
    const unsigned char* chunk[kMaxDma];
    uint32_t chunk_stride[kMaxDma];  // bytes per page of the chunk's segment
    int n_chunk;                // 16-byte DMA instructions this wave issues per page
};

// The segments of a region are consecutive in chunk order, so chunk c of a lane lies at
// base[s] + 16 c, base[s] = the segment's first byte - 16 * (its first chunk), for the segment s
// that c falls in: the bases and strides are scalars, and each lane picks its own with compares
// and selects -- no divergent branches, a few dozen instructions before the first DMA.  Empty
// segments (a tier of width 0) have equal boundaries and are never picked.
__device__ __forceinline__ void dma_setup(DmaSrc& s, const lf_packed_layer& L, const MfmaLayout& y, int b, int h,
                                          int pbeg, int wave, int lane) {
    const int64_t row0 = tok_row(L, b, h, static_cast<int64_t>(pbeg) * kPage);
    const int na = y.seg_end[2];             // region A chunks
    const int nb_chunks = y.n_chunks - na;   // region B chunks
    const int e0 = y.seg_end[0], e1 = y.seg_end[1];
    const int c_f16 = 288, c_sm = 288 + kPage * L.k_width[3] * 2 / 16;  // region B segment starts
    const auto addr = [](const void* ptr, int64_t bytes, int first_chunk) {
        return reinterpret_cast<uint64_t>(ptr) + static_cast<uint64_t>(bytes) - 16u * static_cast<uint64_t>(first_chunk);
    };
    // region A: Key-code rows K0, K1, K2
    const uint64_t ka0 = addr(L.k_code[0], row0 * L.k_words[0] * 4, 0);
    const uint64_t ka1 = addr(L.k_code[1], row0 * L.k_words[1] * 4, e0);
    const uint64_t ka2 = addr(L.k_code[2], row0 * L.k_words[2] * 4, e1);
    const uint32_t ks0 = kPage * L.k_words[0] * 4, ks1 = kPage * L.k_words[1] * 4, ks2 = kPage * L.k_words[2] * 4;
    // region B: v scale (16 chunks), v min (16), v codes (256), fp16-tier rows, the k_sm_page block
    const uint64_t vb0 = addr(L.v_scale, row0 * 2, 0);
    const uint64_t vb1 = addr(L.v_min, row0 * 2, 16);
    const uint64_t vb2 = addr(L.v_code, row0 * 32, 32);
    const uint64_t vb3 = addr(L.k_value16, row0 * L.k_width[3] * 2, c_f16);
    const uint64_t vb4 = addr(L.k_sm_page, sm_page_idx(L, b, h, pbeg) * 2, c_sm);
    const uint32_t vs3 = kPage * L.k_width[3] * 2, vs4 = 32 * y.nb_int;
    s.n_chunk = 0;
#pragma unroll
    for (int i = 0; i < kMaxDma; ++i) {
        const int j = kWaves * i + wave;
        if (j < y.ja + y.jb) s.n_chunk = i + 1;
        uint64_t src = ka0;
        uint32_t stride = 0;
        if (j < y.ja) {
            const int c = min(64 * j + lane, na - 1);
            src = (c >= e1 ? ka2 : c >= e0 ? ka1 : ka0) + 16u * static_cast<uint32_t>(c);
            stride = c >= e1 ? ks2 : c >= e0 ? ks1 : ks0;
        } else if (j < y.ja + y.jb) {
            const int c = min(64 * (j - y.ja) + lane, nb_chunks - 1);
            src = (c >= c_sm ? vb4 : c >= c_f16 ? vb3 : c >= 32 ? vb2 : c >= 16 ? vb1 : vb0) + 16u * static_cast<uint32_t>(c);
            stride = c >= c_sm ? vs4 : c >= c_f16 ? vs3 : c >= 32 ? kPage * 32 : kPage * 2;
        }
        s.chunk[i] = reinterpret_cast<const unsigned char*>(src);
        s.chunk_stride[i] = stride;
    }
}

// Issue the DMA of page ``page`` into the page slot at LDS address ``slot`` (32-bit): block j
// of region A lands at 1024 j, block j of region B at rawa_bytes + 1024 j = 1024 (ja + j), so
// this wave's i-th instruction (block wave + 4 i overall) lands at 1024 (wave + 4 i).  The
// sources advance one page.
__device__ __forceinline__ void dma_page(DmaSrc& s, uint32_t slot, int wave) {
    // The count passes through an empty asm so the compiler keeps one compare per instruction
    // instead of hoisting per-instruction conditions out of the page loop.
    int n_chunk = __builtin_amdgcn_readfirstlane(s.n_chunk);
    asm volatile("" : "+s"(n_chunk));
    // the destinations are uniform: kept in an SGPR (one scalar add per instruction into M0)
    uint32_t d16 = __builtin_amdgcn_readfirstlane(slot + 1024 * wave);
    asm volatile("" : "+s"(d16));
#pragma unroll
    for (int i = 0; i < kMaxDma; ++i) {
        if (i < n_chunk) {
            dma16(s.chunk[i], d16 + 4096 * i);
            s.chunk[i] += s.chunk_stride[i];
        }
    }
}

// Page preparation, in two halves: prep_load issues the LDS reads of a page's rest buffer
// into registers -- before the previous page's compute, so their latency hides behind it --
// and prep_store converts them into the page's prepared buffer after that compute.
//
// Qs work: wave w takes blocks [w * nbw, (w + 1) * nbw) of the integer tiers (nbw = nb_int / 4
// rounded up), lane = 8 * (block - w * nbw) + head, so a wave's q, scale/min reads and Qs
// writes are consecutive in LDS (no bank conflicts).  Value scale/min: even threads, fp16-tier
// rows: odd threads (token tid / 2).
struct PrepRegs {
    uint32_t vc[4];  // Value-code dwords: word tid % 8 of tokens 4 * (tid / 8) + (k + tid / 8) % 4
    uint32_t vs, vm; // Value scale / min bits of token tid / 2 (used by even tid)
    uint32_t f16[2][2];  // fp16-tier halves of the repack dwords (see F16Map)
    QsRegs qs;       // Qs operands of the lane's first block
};

// The fp16-tier rows ([128][w16] halves in the rest buffer) are repacked into [128][w16p]
// (zero padded to whole 8-half blocks): thread tid builds output dwords tid and tid + 256 from
// two halves each.  Offsets are fixed per layer, so they are computed once.
struct F16Map {
    int src[2];      // byte offset of the dword's first half in the rest buffer (0 when unused)
    int dst[2];      // byte offset of the dword in the prepared buffer (the spare dword past the end)
    uint32_t keep[2];  // 0xffff for each half that exists, else 0
};

__device__ __forceinline__ F16Map f16_map(const LoopY& z, int w16, int tid) {
    F16Map m;
    const int hw = z.w16p >> 1;  // output dwords per token
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int d = tid + 256 * i;
        // d / hw through the reciprocal: (d + 0.5) / hw lies at least 0.5 / hw (>= 1/128) from an
        // integer, far beyond the rounding of the product for d < 512
        const int t = hw ? static_cast<int>((static_cast<float>(d) + 0.5f) * __builtin_amdgcn_rcpf(static_cast<float>(hw))) : 0;
        const int c = hw ? d - t * hw : 0;
        const bool live = hw && t < kPage;
        const bool lo = live && 2 * c < w16, hi = live && 2 * c + 1 < w16;
        m.src[i] = lo ? kRawbF16 + 2 * (t * w16 + 2 * c) : 0;
        m.dst[i] = z.ck_v16 + 4 * (live ? d : kPage * hw);  // past the end: the spare dword after the rows
        m.keep[i] = (lo ? 0xffffu : 0u) | (hi ? 0xffff0000u : 0u);
    }
    return m;
}

__device__ __forceinline__ float beta_lo_of(int tier) { return tier == 0 ? 16.f : tier == 1 ? 256.f : 1024.f; }
__device__ __forceinline__ float beta_hi_of(int tier) { return tier == 0 ? 4.f : tier == 1 ? 16.f : 1024.f; }

__device__ __forceinline__ void prep_load(const LoopY& z, const F16Map& fm, const unsigned char* raw,
                                          const float* qperm, int tid, int wave, PrepRegs& r) {
    // read k of thread (tg, w) takes token 4 tg + (k + tg) % 4: the 32 lanes of a half wave then
    // hit 32 different banks
    const int tg = tid >> 3, w = tid & 7;
    const uint32_t* vc = reinterpret_cast<const uint32_t*>(raw + kRawbVc) + 32 * tg + w;
#pragma unroll
    for (int k = 0; k < 4; ++k) r.vc[k] = vc[8 * ((k + tg) & 3)];
    // Every read below is unconditional (addresses clamped into the buffers), so the whole
    // fetch goes out in one batch without a wait; what a thread does not need it ignores.
    r.vs = reinterpret_cast<const uint16_t*>(raw + kRawbVs)[tid >> 1];
    r.vm = reinterpret_cast<const uint16_t*>(raw + kRawbVm)[tid >> 1];
    // both halves of each repack dword: two 2-byte reads (rows of odd width are 2-byte aligned);
    // the high half of the last column reads the next row or padding and is masked off later
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(raw + fm.src[i]);
        r.f16[i][0] = h[0];
        r.f16[i][1] = h[1];
    }
    const int lane = tid & 63, n = lane & 7, j = lane >> 3;
    const int nbw = (z.nb_int + 3) >> 2, gb = min(wave * nbw + j, z.nb_int - 1);
    qs_fetch(qperm + gb * 64 + 4 * n, raw + z.rawb_sm + 32 * gb, r.qs);
}

// Integer-tier Qs and bias of head n for block gb from fetched operands.
__device__ __forceinline__ float qs_block(const LoopY& z, const QsRegs& r, half8* qs, int gb, int n) {
    const int tier = gb >= 4 * z.kf2 ? 2 : gb >= 4 * z.kf1 ? 1 : 0;
    half8* hi = qs + gb * 16 + n;
    half8* lo = qs + gb * 16 + 8 + n;
    return qs_math(r, hi, lo, beta_lo_of(tier), beta_hi_of(tier));
}

// Finish the page: fetched registers ``r`` (and, for what they do not hold, the page's rest
// buffer ``raw``) into prepared buffer ``ck`` (all threads).
__device__ __forceinline__ void prep_store(const LoopY& z, const F16Map& fm, const PrepRegs& r, const unsigned char* raw,
                                           unsigned char* ck, const float* qperm, int g, int w16, int tid, int wave) {
    const int lane = tid & 63;
    {
        // Value codes: dwords (group tg, word w, tokens 0..3) -> byte columns.  The reads came
        // in token order rotated by tg % 4, so each column comes out rotated by as many bytes.
        const int tg = tid >> 3, w = tid & 7;
        const uint32_t rot = (32 - 8 * (tg & 3)) & 31;
        uint32_t o[4];
        byte_transpose4(r.vc[0], r.vc[1], r.vc[2], r.vc[3], o);
        uint32_t* vt = reinterpret_cast<uint32_t*>(ck + kCkVt);
#pragma unroll
        for (int k = 0; k < 4; ++k) vt[tg * 36 + k * 8 + w] = __builtin_amdgcn_alignbit(o[k], o[k], rot);
    }
    {
        // Value scale and the per-token constant vmin - 4 * vscale (4: the offset of the
        // Value-code unpack) of token tid / 2, stored by both threads of the pair (the same
        // values; no branch, so the reads above stay in one batch)
        const int t = tid >> 1;
        const float s = f16_to_f32(static_cast<uint16_t>(r.vs));
        const float mid = fmaf(-4.f, s, f16_to_f32(static_cast<uint16_t>(r.vm)));
        reinterpret_cast<float*>(ck + kCkVsc)[t] = s;
        reinterpret_cast<float*>(ck + kCkVmid)[t] = mid;
    }
    // fp16-tier repack: dwords tid and tid + 256, then (rows wider than 8) the rest
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<uint32_t*>(ck + fm.dst[i]) = (r.f16[i][0] | (r.f16[i][1] << 16)) & fm.keep[i];
    const int hw = z.w16p >> 1;
    if (kPage * hw > 512) {
        for (int d = tid + 512; d < kPage * hw; d += 256) {
            const int t = d / hw, c = d - t * hw;
            const uint16_t* h = reinterpret_cast<const uint16_t*>(raw + kRawbF16) + t * w16 + 2 * c;
            const uint32_t lo = 2 * c < w16 ? h[0] : 0u, hi = 2 * c + 1 < w16 ? h[1] : 0u;
            reinterpret_cast<uint32_t*>(ck + z.ck_v16)[d] = lo | (hi << 16);
        }
    }
    // Qs of the integer tiers and this wave's share of the bias.  The fp16 tier's Qs (plain q)
    // is set once.  Every lane computes and writes its (clamped) block: lanes past the wave's
    // share or past the last block rewrite another lane's block with the same values, rows of
    // heads >= g get the zeros they hold (their q is 0); only owned lanes count in the bias.
    const int n = lane & 7, j = lane >> 3;
    const int nbw = (z.nb_int + 3) >> 2;
    half8* qs = reinterpret_cast<half8*>(ck + kCkQs);
    const int gb_own = wave * nbw + j;
    float bsum = qs_block(z, r.qs, qs, min(gb_own, z.nb_int - 1), n);
    if (!(n < g && j < nbw && gb_own < z.nb_int)) bsum = 0.f;
    if (nbw > 8) {
        for (int jj = j + 8; jj < nbw; jj += 8) {
            const int gb2 = wave * nbw + jj;
            if (n < g && gb2 < z.nb_int) {
                QsRegs q2;
                qs_fetch(qperm + gb2 * 64 + 4 * n, raw + z.rawb_sm + 32 * gb2, q2);
                bsum += qs_block(z, q2, qs, gb2, n);
            }
        }
    }
    // sum over the wave's lanes of head n (lanes n + 8 i): row_ror:8, then across the 4 rows
    bsum += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, bsum), 0x128, 0xf, 0xf, false));
    bsum = rows_sum(bsum);
    if (lane < 8) reinterpret_cast<float*>(ck + kCkBias)[4 * lane + wave] = bsum;
}

// q of the workgroup's rows row0 .. row0 + g - 1, scaled into the log2 domain, into qlin [8][128]
// (0 for rows >= g).
__device__ __forceinline__ void load_q(const DecodeParams& p, int b, int h, int row0, int g, float* qlin, int tid) {
    const lf_decode_args& A = p.A;
    for (int e = tid; e < 8 * kD; e += kThreads) {
        const int n = e / kD, c = e % kD;
        qlin[e] = n < g ? load_as_f32(A.query, (static_cast<int64_t>(b) * A.n_q + h * p.g + row0 + n) * kD + c,
                                      A.q_dtype) * p.qscale
                        : 0.f;
    }
}

// Score operands of one page for one lane: Key-code rows of the three integer tiers, the
// prepared fp16-tier rows and Qs, the lane's two token rows and MFMA coordinates.
struct KTiles {
    const uint32_t* k0;
    const uint32_t* k1;
    const uint32_t* k2;
    const unsigned char* v16;
    const half8* qs;
    int kw0, kw1, kw2, w16p, tok0, tok1, kb, n16;
};

// S^T of the lane's two 16-token tiles, any K-step counts.  Integer tiers read up to 7 dwords
// past their segment (inside the LDS allocation): those blocks have Qs == 0 and unpack to
// finite values.
__device__ __forceinline__ void score_tiles(const KTiles& t, const LoopY& z, const UnpackBits& kv, float4v& acc0,
                                            float4v& acc1) {
    acc0 = float4v{0.f, 0.f, 0.f, 0.f};
    acc1 = float4v{0.f, 0.f, 0.f, 0.f};
    for (int s2 = 0; s2 < z.kst0 / 2; ++s2) {
        const uint32_t wa = t.k0[t.tok0 * t.kw0 + 4 * s2 + t.kb];
        const uint32_t wb = t.k0[t.tok1 * t.kw0 + 4 * s2 + t.kb];
        const half8 bq0 = t.qs[(8 * s2 + t.kb) * 16 + t.n16];
        const half8 bq1 = t.qs[(8 * s2 + 4 + t.kb) * 16 + t.n16];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack2<0>(wa, kv), bq0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack2<0>(wb, kv), bq0, acc1, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack2<1>(wa, kv), bq1, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack2<1>(wb, kv), bq1, acc1, 0, 0, 0);
    }
    for (int s = 0; s < z.kst1; ++s) {
        const half8 bq = t.qs[(4 * (z.kst0 + s) + t.kb) * 16 + t.n16];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack4(t.k1[t.tok0 * t.kw1 + 4 * s + t.kb], kv), bq, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack4(t.k1[t.tok1 * t.kw1 + 4 * s + t.kb], kv), bq, acc1, 0, 0, 0);
    }
    for (int s = 0; s < z.kst2; ++s) {
        const int w0 = 2 * (4 * s + t.kb);
        const half8 bq = t.qs[(4 * (z.kf2 + s) + t.kb) * 16 + t.n16];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack8(t.k2[t.tok0 * t.kw2 + w0], t.k2[t.tok0 * t.kw2 + w0 + 1]), bq,
                                                      acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack8(t.k2[t.tok1 * t.kw2 + w0], t.k2[t.tok1 * t.kw2 + w0 + 1]), bq,
                                                      acc1, 0, 0, 0);
    }
    for (int s = 0; s < z.kst3; ++s) {
        const int col = 8 * (4 * s + t.kb);
        const bool ok = col < t.w16p;
        const int cc = ok ? col : 0;
        const uint4 ra = *reinterpret_cast<const uint4*>(t.v16 + 2 * (t.tok0 * t.w16p + cc));
        const uint4 rb = *reinterpret_cast<const uint4*>(t.v16 + 2 * (t.tok1 * t.w16p + cc));
        const uint4 ua = ok ? ra : uint4{0, 0, 0, 0}, ub = ok ? rb : uint4{0, 0, 0, 0};
        const half8 bq = t.qs[(4 * (z.kf3 + s) + t.kb) * 16 + t.n16];
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ua), bq, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ub), bq, acc1, 0, 0, 0);
    }
}

// The same for K-step counts known at compile time (P2 int2 step pairs, S1 int4, S2 int8, S3
// fp16 steps): every LDS read of the page is issued before the first unpack, so the page
// costs one LDS round trip instead of one per step.
template <int P2, int S1, int S2, int S3>
__device__ __forceinline__ void score_tiles_fixed(const KTiles& t, const UnpackBits& kv, float4v& acc0, float4v& acc1) {
    constexpr int F1 = 2 * P2, F2 = F1 + S1, F3 = F2 + S2;  // first K-step of each tier
    uint32_t w2[P2][2], w4[S1 > 0 ? S1 : 1][2], w8[S2 > 0 ? S2 : 1][2][2];
    uint4 wf[S3 > 0 ? S3 : 1][2];
    half8 q2[P2][2], q4[S1 > 0 ? S1 : 1], q8[S2 > 0 ? S2 : 1], qf[S3 > 0 ? S3 : 1];
    const int toks[2] = {t.tok0, t.tok1};
#pragma unroll
    for (int s2 = 0; s2 < P2; ++s2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) w2[s2][i] = t.k0[toks[i] * t.kw0 + 4 * s2 + t.kb];
        q2[s2][0] = t.qs[(8 * s2 + t.kb) * 16 + t.n16];
        q2[s2][1] = t.qs[(8 * s2 + 4 + t.kb) * 16 + t.n16];
    }
#pragma unroll
    for (int s = 0; s < S1; ++s) {
#pragma unroll
        for (int i = 0; i < 2; ++i) w4[s][i] = t.k1[toks[i] * t.kw1 + 4 * s + t.kb];
        q4[s] = t.qs[(4 * (F1 + s) + t.kb) * 16 + t.n16];
    }
#pragma unroll
    for (int s = 0; s < S2; ++s) {
        const int w0 = 2 * (4 * s + t.kb);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            w8[s][i][0] = t.k2[toks[i] * t.kw2 + w0];
            w8[s][i][1] = t.k2[toks[i] * t.kw2 + w0 + 1];
        }
        q8[s] = t.qs[(4 * (F2 + s) + t.kb) * 16 + t.n16];
    }
    bool okf[S3 > 0 ? S3 : 1];
#pragma unroll
    for (int s = 0; s < S3; ++s) {
        const int col = 8 * (4 * s + t.kb);
        okf[s] = col < t.w16p;
        const int cc = okf[s] ? col : 0;
#pragma unroll
        for (int i = 0; i < 2; ++i) wf[s][i] = *reinterpret_cast<const uint4*>(t.v16 + 2 * (toks[i] * t.w16p + cc));
        qf[s] = t.qs[(4 * (F3 + s) + t.kb) * 16 + t.n16];
    }
    float4v acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int s2 = 0; s2 < P2; ++s2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack2<0>(w2[s2][i], kv), q2[s2][0], acc[i], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack2<1>(w2[s2][i], kv), q2[s2][1], acc[i], 0, 0, 0);
    }
#pragma unroll
    for (int s = 0; s < S1; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i) acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack4(w4[s][i], kv), q4[s], acc[i], 0, 0, 0);
#pragma unroll
    for (int s = 0; s < S2; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(unpack8(w8[s][i][0], w8[s][i][1]), q8[s], acc[i], 0, 0, 0);
#pragma unroll
    for (int s = 0; s < S3; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint4 u = okf[s] ? wf[s][i] : uint4{0, 0, 0, 0};
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, u), qf[s], acc[i], 0, 0, 0);
        }
    acc0 = acc[0];
    acc1 = acc[1];
}

// Residual pass on the matrix cores, for 2-byte tail and new-token rows of one dtype (Bf: bf16,
// else fp16) with 16-byte aligned rows.  The residual is the tl tail rows followed by the new
// tokens (q_len of them, or none), taken as dense chunks of 128 tokens: token tt < tl is tail row
// tt, token tl + j new token j, tokens past them are masked (rows read for them are stored rows:
// new token 0, or tail row 0 when there is none, so every value read is a stored one).  New token
// j is masked for query rows whose token index (row % q_len) is below j -- the right-aligned
// causal mask of reference.py:18-27,48 (with one new token nothing is masked but the chunk's
// end).  Wave w takes tokens c0 + 32w .. + 31 of each chunk as two 16-row tiles:
//   scores  S^T = K . Qb^T: the A operand (lane: token row n16, channels 32 kb + 8 s .. + 7 of
//           K-step s) straight from global memory; Qb = the LDS query (q * scaling * log2 e)
//           split hi (columns 0..7) / lo (columns 8..15), recombined by one DPP add;
//   values  O = P . V with P = 2^(s - m) split hi (rows 0..7) / lo (rows 8..15): the score
//           accumulator layout is the A-operand layout; the wave's 32 V rows arrive by LDS-DMA
//           into its own 8 KB of ``vst`` and each lane gathers its 8 tokens of one channel.
// A chunk after the first (only when tl + q_len > 128) rescales the wave's running (m, l, O) by
// 2^(m_old - m_new).  The wave's (m, l, o) go to partial slot ``rw`` with a zero midpoint term.
// ``vst`` may overlap partial slots other than 0..3: the stores wait for every wave's last V read.
template <bool Bf>
__device__ __forceinline__ void residual_mfma(const DecodeParams& p, int b, int h, int row0, int g, int rw, int tl,
                                              float* qlin, float* red, float* wstat, float* alpha_lds,
                                              unsigned char* vst, int tid) {
    using T8 = typename std::conditional<Bf, bf16x8, half8>::type;
    const lf_decode_args& A = p.A;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15, kb = lane >> 4;
    const bool has_new = A.k_new != nullptr;
    const int q_len = p.q_len;
    const int n_res = tl + (has_new ? q_len : 0);
    const int64_t bh = static_cast<int64_t>(b) * p.L.n_kv + h;
    const uint16_t* tk = static_cast<const uint16_t*>(A.tail_k) + bh * A.tail_cap * kD;
    const uint16_t* tv = static_cast<const uint16_t*>(A.tail_v) + bh * A.tail_cap * kD;
    // new token 0 of this (b, h): k_new / v_new are [batch][n_kv][q_len][128]
    const uint16_t* fk = has_new ? static_cast<const uint16_t*>(A.k_new) + bh * q_len * kD : tk;
    const uint16_t* fv = has_new ? static_cast<const uint16_t*>(A.v_new) + bh * q_len * kD : tv;
    // the row of residual token tt (a stored row for masked tokens)
    auto row_of = [&](const uint16_t* tail, const uint16_t* fresh, int tt) -> const uint16_t* {
        return tt < tl ? tail + static_cast<int64_t>(tt) * kD : tt < n_res ? fresh + static_cast<int64_t>(tt - tl) * kD : fresh;
    };
    // token index of the query row in score column n16 (lanes n16 < 8 hold the hi + lo sums)
    const int tq = (row0 + (n16 & 7)) % q_len;
    float O[8][4];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[nt][r] = 0.f;
    float mx = -__builtin_inff(), lsum = 0.f;
    if (n_res > 0) {  // uniform over the workgroup
        T8 bq[4];
        for (int c0 = 0; c0 < n_res; c0 += kPage) {  // uniform over the workgroup
            // V rows by LDS-DMA: instruction i moves rows 32 w + 4 i .. + 3 (16 lanes per row)
            const uint32_t vbase = lds_addr(vst) + 8192 * wave;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int tt = c0 + 32 * wave + 4 * i + (lane >> 4);
                dma16(reinterpret_cast<const unsigned char*>(row_of(tv, fv, tt) + 8 * (lane & 15)), vbase + 1024 * i);
            }
            uint4 ka[2][4];
#pragma unroll
            for (int tile = 0; tile < 2; ++tile) {
                const int tt = c0 + 32 * wave + 16 * tile + n16;
                const uint4* row = reinterpret_cast<const uint4*>(row_of(tk, fk, tt) + 32 * kb);
#pragma unroll
                for (int s = 0; s < 4; ++s) ka[tile][s] = row[s];
            }
            if (c0 == 0) {
                load_q(p, b, h, row0, g, qlin, tid);  // its wait also covers the K and V loads: one round trip
                __syncthreads();                      // q in LDS
                const float4* q4 = reinterpret_cast<const float4*>(qlin + (n16 & 7) * kD + 32 * kb);
                const bool lo = n16 >= 8;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const float4 a = q4[2 * s], c = q4[2 * s + 1];
                    const float x[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        if constexpr (Bf) {
                            const __bf16 hi = static_cast<__bf16>(x[j]);
                            bq[s][j] = lo ? static_cast<__bf16>(x[j] - static_cast<float>(hi)) : hi;
                        } else {
                            const _Float16 hi = static_cast<_Float16>(x[j]);
                            bq[s][j] = lo ? static_cast<_Float16>(x[j] - static_cast<float>(hi)) : hi;
                        }
                    }
                }
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this chunk's V rows have landed
            }
            float4v acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                if constexpr (Bf) {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[0][s]), bq[s], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[1][s]), bq[s], acc1, 0, 0, 0);
                } else {
                    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ka[0][s]), bq[s], acc0, 0, 0, 0);
                    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, ka[1][s]), bq[s], acc1, 0, 0, 0);
                }
            }
            // hi + lo columns (lanes n16 < 8: row n16, tokens 4 kb + r of each tile); masked -inf
            const int tb = c0 + 32 * wave + 4 * kb;
            const float accs[8] = {acc0[0], acc0[1], acc0[2], acc0[3], acc1[0], acc1[1], acc1[2], acc1[3]};
            float sv[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int xi = __builtin_bit_cast(int, accs[r]);
                const float sum = accs[r] + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, xi, 0x108, 0xf, 0xf, true));
                const int tt = tb + (r & 3) + 16 * (r >> 2);
                sv[r] = tt < n_res && tt - tl <= tq ? sum : -__builtin_inff();
            }
            float cm = sv[0];
#pragma unroll
            for (int i = 1; i < 8; ++i) cm = fmaxf(cm, sv[i]);
            cm = rows_max(cm);
            const float m_new = fmaxf(mx, cm);
            const float moff = m_new == -__builtin_inff() ? 0.f : m_new;
            if (c0 > 0) {
                // rescale the running sums: O row 4 kb + r holds row (4 kb + r) % 8 of the tile,
                // whose factor lane (kb 0, n16 = that row) publishes
                const float alpha = __builtin_amdgcn_exp2f(mx - moff);
                lsum *= alpha;
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
            mx = m_new;
            float pp[8], psum = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                pp[i] = __builtin_amdgcn_exp2f(sv[i] - moff);
                psum += pp[i];
            }
            lsum += rows_sum(psum);
            // A operand: k = 8 kb + j <-> token 4 kb + j (tile 0, j < 4) / 16 + 4 kb + j - 4 (tile 1);
            // hi in lanes n16 < 8, lo (moved 8 lanes up) in lanes n16 >= 8
            uint32_t ahi[4], alo[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float x0 = pp[2 * j], x1 = pp[2 * j + 1];
                uint16_t hb[2], lb[2];
                if constexpr (Bf) {
                    const __bf16 h0 = static_cast<__bf16>(x0), h1 = static_cast<__bf16>(x1);
                    const __bf16 l0 = static_cast<__bf16>(x0 - static_cast<float>(h0)), l1 = static_cast<__bf16>(x1 - static_cast<float>(h1));
                    hb[0] = __builtin_bit_cast(uint16_t, h0); hb[1] = __builtin_bit_cast(uint16_t, h1);
                    lb[0] = __builtin_bit_cast(uint16_t, l0); lb[1] = __builtin_bit_cast(uint16_t, l1);
                } else {
                    const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
                    const _Float16 l0 = static_cast<_Float16>(x0 - static_cast<float>(h0)), l1 = static_cast<_Float16>(x1 - static_cast<float>(h1));
                    hb[0] = __builtin_bit_cast(uint16_t, h0); hb[1] = __builtin_bit_cast(uint16_t, h1);
                    lb[0] = __builtin_bit_cast(uint16_t, l0); lb[1] = __builtin_bit_cast(uint16_t, l1);
                }
                ahi[j] = hb[0] | (static_cast<uint32_t>(hb[1]) << 16);
                alo[j] = lb[0] | (static_cast<uint32_t>(lb[1]) << 16);
            }
            uint4 au;
            au.x = __builtin_amdgcn_update_dpp(ahi[0], alo[0], 0x118, 0xf, 0xc, false);
            au.y = __builtin_amdgcn_update_dpp(ahi[1], alo[1], 0x118, 0xf, 0xc, false);
            au.z = __builtin_amdgcn_update_dpp(ahi[2], alo[2], 0x118, 0xf, 0xc, false);
            au.w = __builtin_amdgcn_update_dpp(ahi[3], alo[3], 0x118, 0xf, 0xc, false);
            // this wave's V rows have landed (the first chunk's barrier waited for all of its vector
            // memory, later chunks wait above)
            const uint16_t* vs = reinterpret_cast<const uint16_t*>(vst + 8192 * wave);
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                const int c = 16 * nt + n16;
                uint16_t e[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) e[j] = vs[(4 * kb + (j & 3) + 16 * (j >> 2)) * kD + c];
                const uint4 bu = {e[0] | (static_cast<uint32_t>(e[1]) << 16), e[2] | (static_cast<uint32_t>(e[3]) << 16),
                                  e[4] | (static_cast<uint32_t>(e[5]) << 16), e[6] | (static_cast<uint32_t>(e[7]) << 16)};
                float4v o4 = {O[nt][0], O[nt][1], O[nt][2], O[nt][3]};
                if constexpr (Bf)
                    o4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, au), __builtin_bit_cast(bf16x8, bu), o4, 0, 0, 0);
                else
                    o4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, au), __builtin_bit_cast(half8, bu), o4, 0, 0, 0);
                O[nt][0] = o4[0]; O[nt][1] = o4[1]; O[nt][2] = o4[2]; O[nt][3] = o4[3];
            }
        }
        // rows r (hi) + r + 8 (lo): lanes kb < 2 hold rows 4 kb + r
#pragma unroll
        for (int nt = 0; nt < 8; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) O[nt][r] = halves_sum(O[nt][r]);
    }
    __syncthreads();  // every wave's V reads are done (vst may overlap partial slots)
    if (kb < 2) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(rw * 8 + 4 * kb + r) * kD + 16 * nt + n16] = O[nt][r];
    }
    if (kb == 0 && n16 < 8) {
        wstat[(rw * 3 + 0) * 8 + n16] = mx;
        wstat[(rw * 3 + 1) * 8 + n16] = lsum;
        wstat[(rw * 3 + 2) * 8 + n16] = 0.f;
    }
    __syncthreads();
}


// Merge NP wave partials (m, l, mid of each head in wstat [NP][3][8], o in red [NP][8][128])
// into the item's partial record of each of the g rows: thread tid takes row tid / 32, channels
// 4 (tid % 32) .. + 3.  Every LDS read of a thread goes out in one batch (the partials of a
// head are the same for the 32 threads of a half wave: broadcast reads), then one exp2 per
// partial, then the stores.
template <int NP>
__device__ __forceinline__ void merge_partials(const DecodeParams& p, int item, int h, int row0, int g,
                                               const float* wstat, const float* red, int tid) {
    const int i = tid >> 5, c4 = 4 * (tid & 31);
    if (i >= g) return;
    float mw[NP], lw[NP], dw[NP];
    float4 ow[NP];
#pragma unroll
    for (int w = 0; w < NP; ++w) {
        mw[w] = wstat[(w * 3 + 0) * 8 + i];
        lw[w] = wstat[(w * 3 + 1) * 8 + i];
        dw[w] = wstat[(w * 3 + 2) * 8 + i];
        ow[w] = *reinterpret_cast<const float4*>(red + (w * 8 + i) * kD + c4);
    }
    float M = mw[0];
#pragma unroll
    for (int w = 1; w < NP; ++w) M = fmaxf(M, mw[w]);
    float4 o = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
    if (M != -__builtin_inff()) {
#pragma unroll
        for (int w = 0; w < NP; ++w) {
            const float sc = __builtin_amdgcn_exp2f(mw[w] - M);
            o.x = fmaf(sc, ow[w].x + dw[w], o.x);
            o.y = fmaf(sc, ow[w].y + dw[w], o.y);
            o.z = fmaf(sc, ow[w].z + dw[w], o.z);
            o.w = fmaf(sc, ow[w].w + dw[w], o.w);
            l = fmaf(sc, lw[w], l);
        }
    }
    // records are (D + 2) floats: 8-byte aligned, so the four channels go out as two float2
    float* rec = part_rec(p, item, h, row0 + i);
    *reinterpret_cast<float2*>(rec + c4) = float2{o.x, o.y};
    *reinterpret_cast<float2*>(rec + c4 + 2) = float2{o.z, o.w};
    if (c4 == 0) *reinterpret_cast<float2*>(rec + kD) = float2{M, l};
}

__global__ __launch_bounds__(kThreads, 2) void decode_mfma_kernel(MfmaParams mp) {
    // The argument block before the inline plan, and this workgroup's inline work record (the
    // launch uses a 2-D grid (n_kv, items) whenever the record is inline, so the item is
    // blockIdx.y; otherwise the slot read is ignored).
    const i32x4 rec_arg = prefetch_args_rec4<offsetof(MfmaParams, work_inline)>(
        static_cast<uint32_t>(offsetof(MfmaParams, work_inline)) + 16u * min(blockIdx.y, LF_INLINE_WORK - 1u));
    const DecodeParams& p = mp.p;
    const MfmaLayout& y = mp.y;
    const UnpackBits kv = vgpr_bits(mp.k);
    const lf_packed_layer& L = p.L;
    const lf_decode_args& A = p.A;
    // Item-major: workgroup id = item * n_kv + h, so the work list's order is the dispatch
    // order (the host's split plan relies on it).  With more than 8 query rows per kv head the
    // rows come in tiles of 8, one workgroup each: the n_rt tiles of (item, h) pair u take ids
    // ((u / 8) * n_rt + rt) * 8 + u % 8.  Workgroup ids go round-robin over the 8 XCDs, so a
    // pair's tiles run on one XCD, close together in time, and its later tiles read the pages
    // from that XCD's L2; ids past the last pair (the grid is padded to whole groups of 8 pairs)
    // return at once.
    const int n_kv = L.n_kv;
    const int n_rt = mp.n_rt;
    int item, h, rt = 0;
    if (n_rt == 1) {
        // grid (n_kv, items): the linear id item * n_kv + h without a division (a plan of more
        // than 65535 items comes as a 1-D grid of item * n_kv + h)
        if (gridDim.x == static_cast<unsigned>(n_kv)) {
            item = blockIdx.y;
            h = blockIdx.x;
        } else {
            item = blockIdx.x / n_kv;
            h = blockIdx.x - item * n_kv;
        }
    } else {
        const int x8 = static_cast<int>(blockIdx.x >> 3);
        const int grp = x8 / n_rt;
        rt = x8 - grp * n_rt;
        const int u = 8 * grp + static_cast<int>(blockIdx.x & 7);
        if (u >= A.n_work * n_kv) return;
        item = u / n_kv;
        h = u - item * n_kv;
    }
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n16 = lane & 15;  // MFMA column / row index
    const int kb = lane >> 4;   // lane group
    const int row0 = 8 * rt;              // this tile's rows row0 .. row0 + g - 1 of the kv head's p.g
    const int g = min(8, p.g - row0);
    // The work record through the constant address space: one scalar load (the item is uniform),
    // which skips the vector memory pipeline's longer round trip in the prologue's dependent
    // chain.  The list is written before the launch, so the scalar cache (invalidated at
    // dispatch) cannot hold a stale copy.
    typedef const __attribute__((address_space(4))) i32x4 ci32x4;
    const i32x4 rec = mp.inline_work ? rec_arg : ((ci32x4*)A.work)[item];
    const int b = rec[0];
    const int pbeg = rec[1];
    const int pend = rec[2];
    const int kind = rec[3] & 0xff;
    // the item's partial slot: kind bits 8.. hold slot + 1 when the plan lists its items out of
    // slot order (any value past the workspace's n_work falls back to the item's own index)
    const int part_slot = static_cast<unsigned>(rec[3] >> 8) - 1u < static_cast<unsigned>(A.n_work) ? (rec[3] >> 8) - 1 : item;
    // Tier-table entries of this thread's Key-slot block (used by items with pages, below): they
    // depend only on the kv head, so their loads go out while the work record is in flight.  Thread tid owns block gb = tid / 4 (K-step gb / 4); tier_index entries
    // are read whatever the tier count, which decides afterwards which are real slots.
    const int gb = tid >> 2, n0 = 2 * (tid & 3);
    const int i = gb >> 2;
    const bool own = i < y.kst[0] + y.kst[1] + y.kst[2] + y.kst[3];
    const int tier = i >= y.kfirst[3] ? 3 : i >= y.kfirst[2] ? 2 : i >= y.kfirst[1] ? 1 : 0;
    const int lb = gb - 4 * sel4(y.kfirst, tier);
    const bool live = own && block_live(L, tier, lb);  // live: the tier has width > 0
    const int width = sel4(L.k_width, tier);
    int count = 0;
    int craw[8];
    int slot[8];
    block_slots(tier, lb, slot);
    if (live) {
        // global-memory pointers again (the SGPR pin of sel4 hides where they came from; a flat
        // load would also count against lgkmcnt, which every LDS wait below waits for)
        typedef const __attribute__((address_space(1))) int32_t gint;
        const gint* tix = (const gint*)sel4(L.tier_index, tier) + h * width;
        count = ((const gint*)sel4(L.tier_count, tier))[h];
#pragma unroll
        for (int pos = 0; pos < 8; ++pos) craw[pos] = tix[min(slot[pos], width - 1)];
    }

    extern __shared__ __align__(16) unsigned char smem[];
    float* qperm = reinterpret_cast<float*>(smem + y.off_qperm);
    float* small = reinterpret_cast<float*>(smem + y.off_small);
    float* alpha_lds = small;              // [waves][8]: softmax rescale per head
    // Wave partials: slots 0..3 the pages (waves 0..3), slots 4..7 the residual of an item that
    // has both (kind 2; a residual-only item uses slots 0..3).
    float* wstat = small + kWaves * 8;     // [2 * waves][3][8]: m, l, mid per head
    // Aliases of the prepared + raw buffers (free outside the page loop): q [8][128] (the first
    // 4 KB of prepared buffer 0, below its Qs rows), wave partial outputs [2 * waves][8][128],
    // residual probabilities [waves][32][8].
    float* qlin = reinterpret_cast<float*>(smem + y.off_ck);
    float* red = qlin + 8 * kD;
    float* pbuf = red + 2 * kWaves * 8 * kD;

    float O[8][4];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r) O[nt][r] = 0.f;
    float m_run = -__builtin_inff(), l_run = 0.f, mid_run = 0.f;

    if (kind != 1) {
        // ---- pages (kind 0, 2) ----
        const LoopY z = loop_y(y);
        unsigned char* raw0 = smem + y.off_raw;
        unsigned char* ck = smem + y.off_ck;
        const uint32_t raw_lds = lds_addr(smem) + y.off_raw;  // LDS address of page slot 0

        // ---- q permuted into slot order ----
        // K-step i of the layout holds blocks 4i .. 4i+3.  Thread tid owns block gb = tid / 4
        // (K-step gb / 4) for heads 2 (tid % 4) and 2 (tid % 4) + 1, all 8 slot positions: its
        // slots' channels were loaded with the work record (above); q of the workgroup's heads
        // goes whole into qlin [8][128] (the first 4 KB of the prepared buffer), its loads issued
        // right behind the first page's DMA so both land in one round.  After a barrier each
        // thread reads its slots' channels there.
        // Integer tiers go to qperm (0 for padding slots and heads >= g); the fp16 tier's Qs
        // (plain q, hi / lo) goes into the prepared buffer past qlin, which no page rewrites; Qs
        // rows of heads >= g start at 0.  Nothing here waits for the DMA; the page loop's first
        // barrier does.
        DmaSrc ds;
        dma_setup(ds, L, y, b, h, pbeg, wave, lane);
        dma_page(ds, raw_lds, wave);
        // q [8][128] of heads h g .. h g + 7: thread tid takes channels 4 (tid % 32) + 0..3 of
        // head tid / 32 (0 for heads >= g)
        const int qn = tid >> 5, qc0 = 4 * (tid & 31);
        float4 q4 = {0.f, 0.f, 0.f, 0.f};
        if (qn < g) {
            const int64_t qrow = (static_cast<int64_t>(b) * A.n_q + h * p.g + row0 + qn) * kD + qc0;
            // 2-byte q (8-byte aligned): the thread's four channels in one load
            if (A.q_dtype != LF_FP32 && (reinterpret_cast<uintptr_t>(A.query) & 7) == 0) {
                const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(A.query) + qrow);
                const bool bf = A.q_dtype == LF_BF16;
                const uint16_t e[4] = {static_cast<uint16_t>(raw.x), static_cast<uint16_t>(raw.x >> 16),
                                       static_cast<uint16_t>(raw.y), static_cast<uint16_t>(raw.y >> 16)};
                q4.x = (bf ? bf16_to_f32(e[0]) : f16_to_f32(e[0])) * p.qscale;
                q4.y = (bf ? bf16_to_f32(e[1]) : f16_to_f32(e[1])) * p.qscale;
                q4.z = (bf ? bf16_to_f32(e[2]) : f16_to_f32(e[2])) * p.qscale;
                q4.w = (bf ? bf16_to_f32(e[3]) : f16_to_f32(e[3])) * p.qscale;
            } else {
                q4.x = load_as_f32(A.query, qrow + 0, A.q_dtype) * p.qscale;
                q4.y = load_as_f32(A.query, qrow + 1, A.q_dtype) * p.qscale;
                q4.z = load_as_f32(A.query, qrow + 2, A.q_dtype) * p.qscale;
                q4.w = load_as_f32(A.query, qrow + 3, A.q_dtype) * p.qscale;
            }
        }

        {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(ck) + qn * kD + qc0) = q4;
            int chan[8];
#pragma unroll
            for (int pos = 0; pos < 8; ++pos) chan[pos] = live && slot[pos] < count ? craw[pos] : -1;
            __syncthreads();  // qlin complete
            const float* qlin = reinterpret_cast<const float*>(ck);
            // All 16 reads go out unconditionally (channel 0 for a padding slot) and are waited
            // for once: the empty asm takes every value, so the compiler cannot sink a read into
            // the branch of its select (it did: 16 reads, each behind an exec branch and its own
            // LDS wait).
            float qv[2][8];
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int pos = 0; pos < 8; ++pos) qv[r][pos] = qlin[(n0 + r) * kD + max(chan[pos], 0)];
            asm volatile("" : "+v"(qv[0][0]), "+v"(qv[0][1]), "+v"(qv[0][2]), "+v"(qv[0][3]), "+v"(qv[0][4]),
                              "+v"(qv[0][5]), "+v"(qv[0][6]), "+v"(qv[0][7]), "+v"(qv[1][0]), "+v"(qv[1][1]),
                              "+v"(qv[1][2]), "+v"(qv[1][3]), "+v"(qv[1][4]), "+v"(qv[1][5]), "+v"(qv[1][6]),
                              "+v"(qv[1][7]));
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int pos = 0; pos < 8; ++pos) qv[r][pos] = chan[pos] >= 0 && n0 + r < g ? qv[r][pos] : 0.f;
            if (own) {
                _Float16* qs16 = reinterpret_cast<_Float16*>(ck + kCkQs);
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int n = n0 + r;
                    if (i < z.kf3) {
                        float* dst = qperm + gb * 64 + 4 * n;
                        *reinterpret_cast<float4*>(dst) = float4{qv[r][0], qv[r][1], qv[r][2], qv[r][3]};
                        *reinterpret_cast<float4*>(dst + 32) = float4{qv[r][4], qv[r][5], qv[r][6], qv[r][7]};
                    }
                    if (i >= z.kf3 || n >= g) {
                        half8 hi, lo;
#pragma unroll
                        for (int pos = 0; pos < 8; ++pos) {
                            hi[pos] = static_cast<_Float16>(qv[r][pos]);
                            lo[pos] = static_cast<_Float16>(qv[r][pos] - static_cast<float>(hi[pos]));
                        }
                        *reinterpret_cast<half8*>(qs16 + (gb * 16 + n) * 8) = hi;
                        *reinterpret_cast<half8*>(qs16 + (gb * 16 + 8 + n) * 8) = lo;
                    }
                }
            }
        }
        const int w16 = L.k_width[3];
        const F16Map fm = f16_map(z, w16, tid);
        const int kw0 = L.k_words[0], kw1 = L.k_words[1], kw2 = L.k_words[2];
        const int sh = 2 * (n16 & 3);
        const int tok0 = 32 * wave + n16, tok1 = tok0 + 16;
        // Pages in chunks of 64; between chunks the midpoint term is folded into O (below).
        for (int cbeg = pbeg; cbeg < pend; cbeg += 64) {
        const int cend = min(cbeg + 64, pend);
        for (int page = cbeg; page < cend; ++page) {
            const int rel = page - pbeg;
            // Page landed (every wave's share) and page - 1 computed: the prepared buffer and
            // page - 1's slot are free.  (On the first page this also orders the set-up above:
            // qlin, which the prepared buffer aliases, is dead from here on.)
            dma_barrier(0);
            // The preparation is the latency-critical phase (every wave waits for it at the next
            // barrier): it takes issue priority over the other workgroup's compute on the SIMD
            // (c2: 83.8 -> 82.8 us per layer-step in an A/B run).
            __builtin_amdgcn_s_setprio(2);
            // The preparation reads go out first; page + 1's DMA is issued while they are in
            // flight (a DMA instruction can wait for the address unit, shared by the CU's waves).
            const unsigned char* raw = raw0 + (rel & 1) * z.slot_bytes;
            PrepRegs pr;
            prep_load(z, fm, raw + z.rawa_bytes, qperm, tid, wave, pr);
            if (page + 1 < pend) dma_page(ds, raw_lds + ((rel + 1) & 1) * z.slot_bytes, wave);
            prep_store(z, fm, pr, raw + z.rawa_bytes, ck, qperm, g, w16, tid, wave);
            lds_barrier();  // page prepared
            __builtin_amdgcn_s_setprio(0);
            // ---- compute page ``page`` from the prepared buffer and its Key codes ----
            const half8* qs = reinterpret_cast<const half8*>(ck + kCkQs);
            // Value codes of the lane's 8 tokens for channel 16*nt + n16, unpacked just before their
            // product: code bits to mantissa 8..9 under exponent 4, value 4 + c (the offset is
            // folded into the per-token constant); tokens (0, 2) sit at byte bits sh, (1, 3) at 8 + sh
            uint32_t dlo[8], dhi[8];
            {
                const uint32_t* vt = reinterpret_cast<const uint32_t*>(ck + kCkVt);
                const uint4 d0a = *reinterpret_cast<const uint4*>(vt + (8 * wave + kb) * 36 + (n16 >> 2) * 8);
                const uint4 d0b = *reinterpret_cast<const uint4*>(vt + (8 * wave + kb) * 36 + (n16 >> 2) * 8 + 4);
                const uint4 d1a = *reinterpret_cast<const uint4*>(vt + (8 * wave + 4 + kb) * 36 + (n16 >> 2) * 8);
                const uint4 d1b = *reinterpret_cast<const uint4*>(vt + (8 * wave + 4 + kb) * 36 + (n16 >> 2) * 8 + 4);
                dlo[0] = d0a.x; dlo[1] = d0a.y; dlo[2] = d0a.z; dlo[3] = d0a.w;
                dlo[4] = d0b.x; dlo[5] = d0b.y; dlo[6] = d0b.z; dlo[7] = d0b.w;
                dhi[0] = d1a.x; dhi[1] = d1a.y; dhi[2] = d1a.z; dhi[3] = d1a.w;
                dhi[4] = d1b.x; dhi[5] = d1b.y; dhi[6] = d1b.z; dhi[7] = d1b.w;
            }
            // The page's other compute-phase reads go out with the score operands: bias partials,
            // Value scale and midpoint constant of the lane's four tokens.
            const bool lo_lane = n16 >= 8;
            const int tokl = 32 * wave + (lo_lane ? 16 : 0) + 4 * kb;  // the lane's first token
            const float4 bp = reinterpret_cast<const float4*>(ck + kCkBias)[n16 & 7];
            const float4 vs = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(ck + kCkVsc) + tokl);
            const float4 vd = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(ck + kCkVmid) + tokl);
            // Integer tiers read up to 7 dwords past their segment (inside the LDS allocation):
            // those blocks have Qs == 0 and unpack to finite values.
            float4v acc0, acc1;
            {
                const KTiles kt{reinterpret_cast<const uint32_t*>(raw), reinterpret_cast<const uint32_t*>(raw + 16 * z.seg0),
                                reinterpret_cast<const uint32_t*>(raw + 16 * z.seg1), ck + z.ck_v16, qs,
                                kw0, kw1, kw2, z.w16p, tok0, tok1, kb, n16};
                if (z.kst0 == 4 && z.kst1 == 1 && z.kst2 == 1 && z.kst3 == 1)
                    score_tiles_fixed<2, 1, 1, 1>(kt, kv, acc0, acc1);
                else if (z.kst0 == 4 && z.kst1 == 2 && z.kst2 == 1 && z.kst3 == 1)
                    score_tiles_fixed<2, 2, 1, 1>(kt, kv, acc0, acc1);
                else if (z.kst0 == 4 && z.kst1 == 3 && z.kst2 == 1 && z.kst3 == 1)
                    score_tiles_fixed<2, 3, 1, 1>(kt, kv, acc0, acc1);
                else if (z.kst0 == 2 && z.kst1 == 3 && z.kst2 == 1 && z.kst3 == 1)
                    score_tiles_fixed<1, 3, 1, 1>(kt, kv, acc0, acc1);
                else
                    score_tiles(kt, z, kv, acc0, acc1);
            }
            // ---- online softmax (log2 domain), compact: lane n16 < 8 takes tile 0 and lane n16 + 8
            // tile 1 of head n16 % 8, four tokens each; the hi and lo columns meet through
            // row_ror:8.  The accumulator elements are copied to scalars before the DPP move:
            // applied to vector elements directly, this compiler emits one move for all of them.
            float sv[4];
            {
                const float a0[4] = {acc0[0], acc0[1], acc0[2], acc0[3]};
                const float a1[4] = {acc1[0], acc1[1], acc1[2], acc1[3]};
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float own = lo_lane ? a1[r] : a0[r];
                    const int send = __builtin_bit_cast(int, lo_lane ? a0[r] : a1[r]);
                    sv[r] = own + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, send, 0x128, 0xf, 0xf, false));
                }
            }
            const float bias = (bp.x + bp.y) + (bp.z + bp.w);
            // The reference point m_run moves only when some score of the page exceeds it by more
            // than kLazyRescale (probabilities stay below 2^kLazyRescale).  Most pages have no such
            // score: one ballot over the lanes' own maxima then skips the row maxima and the
            // rescale of O and l.  (The first page always takes the long path: m_run = -inf.)
            const float lmx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
            float m_new = m_run;
            if (__builtin_amdgcn_ballot_w64(lmx + bias > m_run + kLazyRescale)) {
                float mx = fmaxf(lmx, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, lmx),
                                                                                              0x128, 0xf, 0xf, false)));
                mx = rows_max(mx);
                const float m_cand = mx + bias;
                const bool grow = m_cand > m_run + kLazyRescale;
                m_new = grow ? m_cand : m_run;
                // Rescale O where a head's max moved: alpha of the 4 output rows this lane holds
                // (rows 4*kb + r, head (4*kb + r) % 8); a same-wave LDS write then read is
                // ordered by the LDS queue.
                const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
                l_run *= alpha;
                mid_run *= alpha;
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
            const float m_off = m_new - bias;  // p = 2^(sv + bias - m_new)
            float pp[4];
            float psum, pmid;
            {
                const float vsa[4] = {vs.x, vs.y, vs.z, vs.w}, vda[4] = {vd.x, vd.y, vd.z, vd.w};
                psum = 0.f;
                pmid = 0.f;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pi = __builtin_amdgcn_exp2f(sv[r] - m_off);
                    psum += pi;
                    pmid = fmaf(pi, vda[r], pmid);
                    pp[r] = pi * vsa[r];
                }
            }
            // A operand of the value product, k order (t0,t2),(t1,t3) of tile 0 then of tile 1 (the
            // lane's tokens 4*kb + r): rows n16 < 8 the hi parts, rows n16 >= 8 the lo parts.  Each
            // lane splits its own four values and swaps the half its partner row needs.
            uint32_t hp[2], lp[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const float x0 = pp[j], x1 = pp[j + 2];
                const _Float16 h0 = static_cast<_Float16>(x0), h1 = static_cast<_Float16>(x1);
                const half2v hv = {h0, h1};
                const half2v lv = {static_cast<_Float16>(x0 - static_cast<float>(h0)),
                                   static_cast<_Float16>(x1 - static_cast<float>(h1))};
                hp[j] = __builtin_bit_cast(uint32_t, hv);
                lp[j] = __builtin_bit_cast(uint32_t, lv);
            }
            uint32_t rv[2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                rv[j] = __builtin_amdgcn_update_dpp(0, lo_lane ? hp[j] : lp[j], 0x128, 0xf, 0xf, false);
            uint4 au;
            au.x = lo_lane ? rv[0] : hp[0];
            au.y = lo_lane ? rv[1] : hp[1];
            au.z = lo_lane ? lp[0] : rv[0];
            au.w = lo_lane ? lp[1] : rv[1];
            const half8 ap = __builtin_bit_cast(half8, au);
            m_run = m_new;
            l_run += psum;
            mid_run += pmid;
            // ---- value product: codes of the lane's 8 tokens, channel 16*nt + n16 ----
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                const uint4 bu = {bfi(dlo[nt] << (8 - sh), kv.m2hi, kv.e4), bfi(dlo[nt] >> sh, kv.m2hi, kv.e4),
                                  bfi(dhi[nt] << (8 - sh), kv.m2hi, kv.e4), bfi(dhi[nt] >> sh, kv.m2hi, kv.e4)};
                float4v o4 = {O[nt][0], O[nt][1], O[nt][2], O[nt][3]};
                o4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap, __builtin_bit_cast(half8, bu), o4, 0, 0, 0);
                O[nt][0] = o4[0]; O[nt][1] = o4[1]; O[nt][2] = o4[2]; O[nt][3] = o4[3];
            }
        }
        // After each 64-page chunk (but the last), fold the midpoint term into O: the Value
        // product accumulates p' * (4 + code) and the offset cancels against
        // sum p * (vmin - 4 vscale) only when the two meet, so the rounding of that
        // cancellation would otherwise grow with the pages of the item (one 256-page item:
        // 3e-4 relative).  Head totals of mid_run (the two tiles, then the 4 lane groups) go
        // to the hi rows 4 * kb + r of lanes kb < 2 through this wave's alpha row, and
        // mid_run restarts at 0.
        if (cend < pend) {
            float mid = mid_run + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mid_run),
                                                                                       0x128, 0xf, 0xf, false));
            mid = rows_sum(mid);
            if (kb == 0 && n16 < 8) alpha_lds[wave * 8 + n16] = mid;
            __builtin_amdgcn_wave_barrier();
            if (kb < 2) {
                const float4 mrow = *reinterpret_cast<const float4*>(alpha_lds + wave * 8 + 4 * kb);
#pragma unroll
                for (int nt = 0; nt < 8; ++nt) {
                    O[nt][0] += mrow.x;
                    O[nt][1] += mrow.y;
                    O[nt][2] += mrow.z;
                    O[nt][3] += mrow.w;
                }
            }
            mid_run = 0.f;
            __builtin_amdgcn_wave_barrier();
        }
        }
        // Reduce l and the midpoint term over the two tiles (lanes n16, n16 ^ 8) and the 4 lane
        // groups of each head.
        l_run += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, l_run), 0x128, 0xf, 0xf, false));
        mid_run += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, mid_run), 0x128, 0xf, 0xf, false));
        l_run = rows_sum(l_run);
        mid_run = rows_sum(mid_run);
        // Rows r (hi, lanes kb 0..1) + rows r+8 (lo, lanes kb 2..3).
#pragma unroll
        for (int nt = 0; nt < 8; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) O[nt][r] = halves_sum(O[nt][r]);
        __syncthreads();  // every wave is done with the buffers that ``red`` aliases
        if (kb < 2) {
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
#pragma unroll
                for (int r = 0; r < 4; ++r) red[(wave * 8 + 4 * kb + r) * kD + 16 * nt + n16] = O[nt][r];
        }
        if (kb == 0 && n16 < 8) {
            wstat[(wave * 3 + 0) * 8 + n16] = m_run;
            wstat[(wave * 3 + 1) * 8 + n16] = l_run;
            wstat[(wave * 3 + 2) * 8 + n16] = mid_run;
        }
        __syncthreads();
    }
    if (kind != 0 && mp.res_mfma != 0) {
        // ---- residual (kind 1, 2) on the matrix cores; its V staging starts at partial slot 4 ----
        const int rw = kind == 2 ? wave + kWaves : wave;
        const int cap = min(A.tail_cap, kPage);
        const int tl = min(max(A.tail_len[b], 0), min(cap, kPage - 1));
        unsigned char* vst = reinterpret_cast<unsigned char*>(red + kWaves * 8 * kD);
        if (mp.res_mfma == 1) residual_mfma<true>(p, b, h, row0, g, rw, tl, qlin, red, wstat, alpha_lds, vst, tid);
        else residual_mfma<false>(p, b, h, row0, g, rw, tl, qlin, red, wstat, alpha_lds, vst, tid);
    } else if (kind != 0) {
        // ---- residual (kind 1, 2): the tail page and the new token (at most page_size tokens) ----
        // One new token (q_len 1; the host sends other calls with a residual to the VALU kernel).
        // VALU: wave w scores tokens 32w..32w+31 (lane % 32 = token, lane / 32 = channel half;
        // q read as float4 from LDS), then accumulates them into channels 2*lane, 2*lane+1.
        // One pass, so each wave's max is final.  For 2-byte residual and new-token rows every
        // global load goes out in one round, before the tail length is known: q (into LDS),
        // the tail length, the lane's tail rows read for every row the residual buffer holds
        // (rows at or past the tail length are then ignored) and the new token's row.
        const int rw = kind == 2 ? wave + kWaves : wave;  // partial slot
        const int cap = min(A.tail_cap, kPage);
        const int64_t bh = static_cast<int64_t>(b) * L.n_kv + h;
        const int t = 32 * wave + (lane & 31);
        const int ch0 = 64 * (lane >> 5);
        const bool has_new = A.k_new != nullptr;
        const bool two_byte = A.tail_dtype != LF_FP32 && (!has_new || A.new_dtype != LF_FP32);
        load_q(p, b, h, row0, g, qlin, tid);
        const int tl = min(max(A.tail_len[b], 0), min(cap, kPage - 1));
        float kv[64];
        float v0[32], v1[32];
        if (two_byte) {
            uint4 kt[8], kn[8];
            uint32_t vt[32], vn = 0;
            const uint16_t* tk = static_cast<const uint16_t*>(A.tail_k) + (bh * A.tail_cap + t) * kD + ch0;
            const uint16_t* tv = static_cast<const uint16_t*>(A.tail_v) + bh * A.tail_cap * kD + 2 * lane;
#pragma unroll
            for (int u = 0; u < 8; ++u) kt[u] = t < cap ? *reinterpret_cast<const uint4*>(tk + 8 * u) : uint4{0, 0, 0, 0};
#pragma unroll
            for (int k = 0; k < 32; ++k)
                vt[k] = 32 * wave + k < cap ? *reinterpret_cast<const uint32_t*>(tv + static_cast<int64_t>(32 * wave + k) * kD) : 0u;
            if (has_new) {
                const uint16_t* nk = static_cast<const uint16_t*>(A.k_new) + bh * kD + ch0;
#pragma unroll
                for (int u = 0; u < 8; ++u) kn[u] = *reinterpret_cast<const uint4*>(nk + 8 * u);
                vn = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(A.v_new) + bh * kD + 2 * lane);
            } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) kn[u] = uint4{0, 0, 0, 0};
            }
            // Token t is the lane's tail row when t < tl, the new token when t == tl.
            const bool from_new = t >= tl;
            const int kdt = from_new ? A.new_dtype : A.tail_dtype;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint4 r = from_new ? kn[u] : kt[u];
                const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const uint16_t x = static_cast<uint16_t>(w[k >> 1] >> (16 * (k & 1)));
                    kv[8 * u + k] = kdt == LF_BF16 ? bf16_to_f32(x) : f16_to_f32(x);
                }
            }
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const int tk2 = 32 * wave + k;
                const uint32_t r = tk2 < tl ? vt[k] : (tk2 == tl ? vn : 0u);
                const int dt = tk2 < tl ? A.tail_dtype : A.new_dtype;
                const uint16_t lo = static_cast<uint16_t>(r & 0xffffu), hi = static_cast<uint16_t>(r >> 16);
                v0[k] = dt == LF_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
                v1[k] = dt == LF_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
            }
        } else {
            // float32 rows: the tail length first, then the rows it selects
            const bool in_tail = t < tl;
            const void* kp = in_tail ? A.tail_k : A.k_new;
            const int kdt = in_tail ? A.tail_dtype : A.new_dtype;
            const int64_t kbase = (in_tail ? (bh * A.tail_cap + t) * kD : bh * kD) + ch0;
#pragma unroll
            for (int i = 0; i < 64; ++i) kv[i] = 0.f;
            if (t < tl + (has_new ? 1 : 0)) {
#pragma unroll
                for (int u = 0; u < 8; ++u) load8_as_f32(kp, kbase + 8 * u, kdt, kv + 8 * u);
            }
#pragma unroll
            for (int k = 0; k < 32; ++k) {
                const int tk2 = 32 * wave + k;
                v0[k] = 0.f;
                v1[k] = 0.f;
                if (tk2 < tl) {
                    v0[k] = load_as_f32(A.tail_v, (bh * A.tail_cap + tk2) * kD + 2 * lane, A.tail_dtype);
                    v1[k] = load_as_f32(A.tail_v, (bh * A.tail_cap + tk2) * kD + 2 * lane + 1, A.tail_dtype);
                } else if (tk2 == tl && has_new) {
                    v0[k] = load_as_f32(A.v_new, bh * kD + 2 * lane, A.new_dtype);
                    v1[k] = load_as_f32(A.v_new, bh * kD + 2 * lane + 1, A.new_dtype);
                }
            }
        }
        const int n_res = tl + (has_new ? 1 : 0);
        const bool act = t < n_res;
        __syncthreads();  // q in LDS
        float s[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4* q4 = reinterpret_cast<const float4*>(qlin + i * kD + ch0);
            float acc = 0.f;
#pragma unroll
            for (int c4 = 0; c4 < 16; ++c4) {
                const float4 q = q4[c4];
                acc = fmaf(q.x, kv[4 * c4], fmaf(q.y, kv[4 * c4 + 1], fmaf(q.z, kv[4 * c4 + 2], fmaf(q.w, kv[4 * c4 + 3], acc))));
            }
            s[i] = acc;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) s[i] += __shfl_xor(s[i], 32, kWave);
        float* pw = pbuf + wave * 32 * 8;  // [32][8]
        float mx[8], pv[8], lt[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) mx[i] = act ? s[i] : -__builtin_inff();
#pragma unroll
        for (int off = 16; off > 0; off >>= 1)
#pragma unroll
            for (int i = 0; i < 8; ++i) mx[i] = fmaxf(mx[i], __shfl_xor(mx[i], off, kWave));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pv[i] = act ? __builtin_amdgcn_exp2f(s[i] - mx[i]) : 0.f;
            lt[i] = pv[i];
        }
#pragma unroll
        for (int off = 16; off > 0; off >>= 1)
#pragma unroll
            for (int i = 0; i < 8; ++i) lt[i] += __shfl_xor(lt[i], off, kWave);
        if (lane < 32) {
#pragma unroll
            for (int i = 0; i < 8; ++i) pw[lane * 8 + i] = pv[i];
        }
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                wstat[(rw * 3 + 0) * 8 + i] = mx[i];
                wstat[(rw * 3 + 1) * 8 + i] = lt[i];
                wstat[(rw * 3 + 2) * 8 + i] = 0.f;
            }
        }
        __builtin_amdgcn_wave_barrier();
        float acc[2][8];
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[cc][i] = 0.f;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                acc[0][i] = fmaf(pw[k * 8 + i], v0[k], acc[0][i]);
                acc[1][i] = fmaf(pw[k * 8 + i], v1[k], acc[1][i]);
            }
        }
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
#pragma unroll
            for (int i = 0; i < 8; ++i) red[(rw * 8 + i) * kD + 2 * lane + cc] = acc[cc][i];
        __syncthreads();
    }

    // ---- merge the wave partials and store this item's partial ----
    if (kind == 2) merge_partials<2 * kWaves>(p, part_slot, h, row0, g, wstat, red, tid);
    else merge_partials<kWaves>(p, part_slot, h, row0, g, wstat, red, tid);
    if (A.commit_new && kind != 0 && rt == 0) commit_new_rows(p, b, h, tid, kThreads);
}

int round_up(int x, int m) { return (x + m - 1) / m * m; }

bool aligned(const void* ptr, uintptr_t a) { return (reinterpret_cast<uintptr_t>(ptr) & (a - 1)) == 0; }

// Host: LDS layout for this layer; false when the shape is outside this kernel.
bool plan_layout(const lf_packed_layer& L, int g, MfmaLayout& y) {
    if (L.head_dim != kD || L.page_size != kPage || L.k_group != kPage || L.bit_v != 2 || L.v_group != kD)
        return false;
    if (g < 1) return false;
    if (L.k_width[0] + L.k_width[1] + L.k_width[2] == 0) return false;
    // the Key scales and mins come from the page-major copy, 16-byte chunks of it
    if (L.k_sm_page == nullptr || !aligned(L.k_sm_page, 16)) return false;
    for (int t = 0; t < 3; ++t)
        if (L.k_width[t] && !aligned(L.k_code[t], 16)) return false;
    if (L.k_width[3] && !aligned(L.k_value16, 16)) return false;
    if (!aligned(L.v_code, 4) || !aligned(L.v_scale, 16) || !aligned(L.v_min, 16)) return false;
    y.kst[0] = 2 * ((L.k_words[0] + 3) / 4);
    y.kst[1] = (L.k_words[1] + 3) / 4;
    y.kst[2] = ((L.k_words[2] + 1) / 2 + 3) / 4;
    y.kst[3] = ((L.k_width[3] + 7) / 8 + 3) / 4;
    int ks = 0;
    for (int t = 0; t < 4; ++t) {
        y.kfirst[t] = ks;
        ks += y.kst[t];
    }
    if (ks > kMaxKSteps) return false;
    y.nb = 4 * ks;
    y.nb_int = 4 * (y.kst[0] + y.kst[1] + y.kst[2]);
    y.w16p = round_up(L.k_width[3], 8);
    int seg = 0;
    for (int t = 0; t < 3; ++t) {
        seg += kPage * L.k_words[t] * 4 / 16;
        y.seg_end[t] = seg;
    }
    // region B (DMA order): v scale, v min, v codes (256 chunks), fp16-tier rows, the page's
    // k_sm_page block (nb_int x 32 bytes; sm_page in lf_common.hpp gives the same block count)
    if (sm_page(L.k_words).nb != y.nb_int) return false;
    y.n_chunks = y.seg_end[2] + 16 + 16 + 256 + kPage * L.k_width[3] * 2 / 16 + 2 * y.nb_int;
    y.ja = (y.seg_end[2] + 63) / 64;
    y.jb = (y.n_chunks - y.seg_end[2] + 63) / 64;
    if (y.ja + y.jb > kMaxDma * kWaves) return false;
    // Key-code buffer: the K0, K1, K2 rows; rest buffer: v scale, v min, Value codes, fp16 tier,
    // the scale/min block.  Every lane of a DMA instruction writes, so both regions are padded to
    // whole 64-chunk blocks (1024 bytes).
    y.rawa_bytes = 1024 * y.ja;
    y.rawb_sm = kRawbF16 + kPage * L.k_width[3] * 2;
    y.rawb_bytes = 1024 * y.jb;
    // prepared buffer: fixed-offset parts, Qs [nb][16][8] fp16 at kCkQs, fp16-tier rows after it
    y.ck_v16 = kCkQs + y.nb * 16 * 16;
    y.ck_bytes = round_up(y.ck_v16 + kPage * y.w16p * 2 + 4, 16);  // + the spare dword of the repack
    y.slot_bytes = y.rawa_bytes + y.rawb_bytes;
    int off = 0;
    y.off_qperm = off;
    off += y.nb_int * 64 * 4;
    y.off_small = off;
    off += (kWaves * 8 + 2 * kWaves * 3 * 8) * 4;  // alpha, wave partial statistics
    off = round_up(off, 16);
    y.off_ck = off;
    off += y.ck_bytes;
    y.off_raw = off;
    off += 2 * y.slot_bytes;
    // q [8][128], wave partial outputs [2 * waves][8][128] and residual probabilities
    // [waves][32][8] alias the prepared buffer and the page slots; so does the matrix-core
    // residual's V staging [waves][32][128] 2-byte rows from partial slot 4 on
    const int alias_bytes = std::max((8 + 2 * kWaves * 8) * kD * 4 + kWaves * 32 * 8 * 4,
                                     (8 + kWaves * 8) * kD * 4 + kWaves * 32 * kD * 2);
    if (off - y.off_ck < alias_bytes) off = y.off_ck + alias_bytes;
    y.lds_bytes = off;
    return y.lds_bytes <= 160 * 1024 - 64;
}

}  // namespace

int launch_decode_mfma(const DecodeParams& p, hipStream_t stream, bool* handled) {
    MfmaParams mp;
    mp.p = p;
    mp.k = UnpackBits{0x00C000C0u, 0x03000300u, 0x003C003Cu, 0x03C003C0u, 0x4C004C00u, 0x44004400u, 0x5C005C00u};
    // The residual pass reads 16-byte Key chunks and 4-byte Value pairs of the tail and new rows.
    const bool rows_aligned = (p.A.tail_cap == 0 || (aligned(p.A.tail_k, 16) && aligned(p.A.tail_v, 4))) &&
                              (!p.A.k_new || (aligned(p.A.k_new, 16) && aligned(p.A.v_new, 4)));
    // The residual on the matrix cores: 2-byte rows of one dtype, every row 16-byte aligned (the
    // V rows go to LDS by 16-byte DMA); otherwise the VALU pass.
    const bool has_tail = p.A.tail_cap > 0, has_new = p.A.k_new != nullptr;
    const int res_dt = has_tail ? p.A.tail_dtype : p.A.new_dtype;
    const bool one_dtype = !has_tail || !has_new || p.A.new_dtype == p.A.tail_dtype;
    const bool rows16 = (!has_tail || (aligned(p.A.tail_k, 16) && aligned(p.A.tail_v, 16))) &&
                        (!has_new || (aligned(p.A.k_new, 16) && aligned(p.A.v_new, 16)));
    mp.res_mfma = (has_tail || has_new) && one_dtype && rows16 && res_dt != LF_FP32 ? (res_dt == LF_BF16 ? 1 : 2) : 0;
    // Several new tokens need the matrix-core residual pass (the VALU pass takes one).
    const bool res_ok = p.q_len == 1 || mp.res_mfma != 0 || (!has_tail && !has_new);
    if (!rows_aligned || !res_ok || !plan_layout(p.L, p.g, mp.y)) {
        *handled = false;
        return LF_OK;
    }
    mp.n_rt = (p.g + 7) / 8;
    const int64_t pairs = static_cast<int64_t>(p.A.n_work) * p.L.n_kv;
    const int64_t blocks = mp.n_rt == 1 ? pairs : (pairs + 7) / 8 * 8 * mp.n_rt;
    if (blocks > 0x7fffffff) return LF_E_SHAPE;
    *handled = true;
    const int rc = allow_dynamic_lds(reinterpret_cast<const void*>(&decode_mfma_kernel), mp.y.lds_bytes);
    if (rc != LF_OK) return rc;
    const bool grid2d = mp.n_rt == 1 && p.A.n_work <= 65535;
    const dim3 grid = grid2d ? dim3(static_cast<unsigned>(p.L.n_kv), static_cast<unsigned>(p.A.n_work))
                             : dim3(static_cast<unsigned>(blocks));
    // the plan inline in the arguments (its slot is blockIdx.y, so only with the 2-D grid)
    mp.inline_work = grid2d && p.A.work_host != nullptr && p.A.n_work <= LF_INLINE_WORK;
    if (mp.inline_work) std::memcpy(mp.work_inline, p.A.work_host, sizeof(int32_t) * 4 * p.A.n_work);
    hipLaunchKernelGGL(decode_mfma_kernel, grid, dim3(kThreads), mp.y.lds_bytes, stream, mp);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return static_cast<int>(err);
    return launch_decode_reduce(p, stream);
}

}  // namespace lf
