/* The fast page packer's arithmetic against IEEE float32 (csrc/pack.hip: raw_scale, div_rn,
 * fast_code, magic_code, value_word_bias), on the CPU with the same operations in the same
 * order: the reference's codes are clamp(rint((x - lo) / s), 0, qmax) with
 * s = clamp((hi - lo) / qmax, 1e-5, 1e5), all float32 (layout.py:12-18).
 * usage: pack_arith_check <groups>; prints the counts and exits 1 on any difference. */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t state = 0x9E3779B97F4A7C15ull;
static uint64_t next(void) { state ^= state << 13; state ^= state >> 7; state ^= state << 17; return state; }
static uint32_t bits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static float bf16(float x) { return from_bits(bits(x) & 0xffff0000u); }
static float clampf(float x, float a, float b) { return fminf(fmaxf(x, a), b); }

/* div_rn: a / s from y = RN(1 / s), the range clamped to FLT_MAX */
static float div_rn(float a, float s, float y) {
    a = fminf(a, FLT_MAX);
    const float q0 = a * y;
    const float r = fmaf(-q0, s, a);
    return fmaf(r, y, q0);
}

int main(int argc, char** argv) {
    const long groups = argc > 1 ? atol(argv[1]) : 100000;
    const int qms[3] = {3, 15, 255};
    long bad = 0, fast = 0, slow = 0, scales = 0;
    /* scale step over ranges of every magnitude (subnormal through overflow) */
    for (long i = 0; i < 20 * groups; ++i) {
        const int qm = qms[i % 3];
        float d = from_bits((uint32_t)(next() & 0x7fffffffu));
        if (isnan(d)) continue;
        if (i % 97 == 0) d = INFINITY;
        const float ref = clampf(d / (float)qm, 1e-5f, 1e5f);
        const float got = clampf(div_rn(d, (float)qm, 1.0f / (float)qm), 1e-5f, 1e5f);
        scales++;
        if (bits(ref) != bits(got) && bad++ < 5) printf("scale: range %a qmax %d: %a vs %a\n", d, qm, got, ref);
    }
    for (long it = 0; it < groups; ++it) {
        const int qm = qms[it % 3];
        const float qmax = (float)qm;
        const int e = (int)(next() % 60) - 30 + ((it % 7 == 0) ? (int)(next() % 40) : 0);
        const float mag = ldexpf(1.0f, e);
        const float off = (next() & 1) ? ldexpf((float)(next() % 1000) - 500.0f, e) : 0.0f;
        float x[32];
        for (int i = 0; i < 32; ++i) {
            x[i] = bf16(off + mag * ((float)((int)(next() % 200001) - 100000) / 100000.0f));
            if (it % 11 == 0 && i < 4) x[i] = bf16(off);
        }
        if (it % 13 == 0) { /* ranges around the 1e5 * qmax boundary of the clamp-free path */
            const float r = 1e5f * qmax * (1.0f + ((float)(int)(next() % 2001) - 1000.0f) * 1e-6f);
            x[0] = bf16(-r * 0.5f);
            x[1] = bf16(r * 0.5f);
        }
        float lo = INFINITY, hi = -INFINITY;
        for (int i = 0; i < 32; ++i) { lo = fminf(lo, x[i]); hi = fmaxf(hi, x[i]); }
        const float s_ref = clampf((hi - lo) / qmax, 1e-5f, 1e5f);
        const float raw = div_rn(hi - lo, qmax, 1.0f / qmax);
        const float s = clampf(raw, 1e-5f, 1e5f);
        if (bits(s) != bits(s_ref)) { if (bad++ < 5) printf("group scale differs\n"); continue; }
        const float y = 1.0f / s;
        const int magic = raw <= 1e5f;
        magic ? fast++ : slow++;
        uint32_t word = 0, word_ref = 0, bias = 0;
        for (int i = 0; i < 16; ++i) bias += 0x4B000000u << (2 * i);
        for (int i = 0; i < 32; ++i) {
            const uint32_t c_ref = (uint32_t)clampf(rintf((x[i] - lo) / s_ref), 0.0f, qmax);
            uint32_t c, t = 0;
            if (magic) {
                const float a = x[i] - lo;
                const float q0 = a * y;
                const float r = fmaf(-q0, s, a);
                t = bits(fmaf(r, y, q0) + 8388608.0f);
                c = t & 0xffu;
            } else {
                c = (uint32_t)clampf(rintf(div_rn(x[i] - lo, s, y)), 0.0f, qmax);
            }
            if (c != c_ref && bad++ < 5) printf("code: qmax %d x %a lo %a s %a: %u vs %u\n", qm, x[i], lo, s, c, c_ref);
            if (qm == 3 && i < 16) {
                word += magic ? t << (2 * i) : c << (2 * i);
                word_ref |= c_ref << (2 * i);
            }
        }
        if (qm == 3 && (magic ? word - bias : word) != word_ref && bad++ < 5) printf("value word differs\n");
    }
    printf("scales %ld, groups %ld (magic %ld, clamped %ld), differences %ld\n", scales, fast + slow, fast, slow, bad);
    return bad != 0;
}
