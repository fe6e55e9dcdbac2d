// Host check of the page-major Key scale/min layout helpers (logitfill_amd/csrc/lf_common.hpp):
// for every tier width and word count the packers and the decode kernel can see, sm_place is the
// inverse of sm_slot, every rank lands at its own position, and positions stay inside the tier's
// blocks.  Prints "ok" or the first failure.
#include <cstdio>
#include "../logitfill_amd/csrc/lf_common.hpp"

int main() {
    for (int t = 0; t < 3; ++t) {
        const int per = 32 >> (t + 1);  // codes per word: 16, 8, 4
        for (int width = 1; width <= 128; ++width) {
            int32_t words[3] = {0, 0, 0};
            words[t] = (width + per - 1) / per;
            const lf::SmPage sp = lf::sm_page(words);
            const int blocks = (t + 1 < 3 ? sp.blk0[t + 1] : sp.nb) - sp.blk0[t];
            static int seen[4096];
            for (int i = 0; i < 8 * blocks; ++i) seen[i] = -1;
            for (int j = 0; j < width; ++j) {
                int lb, pos;
                lf::sm_place(t, j, lb, pos);
                if (lb < 0 || lb >= blocks || pos < 0 || pos >= 8) {
                    printf("tier %d width %d rank %d: block %d pos %d outside %d blocks\n", t, width, j, lb, pos, blocks);
                    return 1;
                }
                if (lf::sm_slot(t, lb, pos) != j) {
                    printf("tier %d rank %d: sm_slot(sm_place) = %d\n", t, j, lf::sm_slot(t, lb, pos));
                    return 1;
                }
                if (seen[8 * lb + pos] >= 0) {
                    printf("tier %d ranks %d and %d share a position\n", t, seen[8 * lb + pos], j);
                    return 1;
                }
                seen[8 * lb + pos] = j;
            }
        }
    }
    printf("ok\n");
    return 0;
}
