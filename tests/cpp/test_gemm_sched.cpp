// Host check of the grouped backward schedule (deepfuse_amd/csrc/gemm_sched.hpp):
// for every parameter set, the units each block walks form an exact
// partition of both problems' units, each block's problem-1 units come in
// increasing order, and the makespan stays within the list-scheduling bound
// (the larger of the problem-0 rounds and the ideal share plus one unit).
// Prints the makespan of the GPT-2 XL backward shapes on 256 CUs.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <vector>

#include "gemm_sched.hpp"

using namespace dfk;

int main() {
    long cases = 0, bad = 0;
    for (int P : {1, 2, 7, 8, 64, 255, 256, 304})
        for (int n0 : {0, 1, 5, 49, 133, 175, 255, 256, 257, 300, 513, 1000})
            for (int c0 : {1, 7, 29, 131})
                for (int n1 : {0, 1, 3, 448, 1000, 1600})
                    for (int c1 : {1, 3, 16, 41, 53}) {
                        const GroupSched s{P, n0, c0, n1, c1};
                        std::vector<int> seen0(n0, 0), seen1(n1, 0);
                        int64_t makespan = 0;
                        for (int b = 0; b < P; ++b) {
                            const int d0 = gs_d0(s, b), d1 = gs_d1(s, b);
                            int prev = -1;
                            for (int r = 0; r < d0 + d1; ++r) {
                                int p, u;
                                gs_unit(s, b, r, p, u);
                                if (p == 0 && u >= 0 && u < n0 && r < d0) {
                                    seen0[u]++;
                                } else if (p == 1 && u > prev && u < n1 && r >= d0) {
                                    seen1[u]++;
                                    prev = u;
                                } else {
                                    ++bad;
                                }
                            }
                            makespan = std::max(makespan, gs_finish(s, b));
                        }
                        for (int v : seen0) bad += v != 1;
                        for (int v : seen1) bad += v != 1;
                        const int64_t work = (int64_t)n0 * c0 + (int64_t)n1 * c1;
                        const int64_t bound = std::max<int64_t>((int64_t)((n0 + P - 1) / P) * c0,
                                                                (work + P - 1) / P + std::max(c0, c1)) + c1;
                        if (makespan > bound) {
                            ++bad;
                            printf("over bound: P=%d n0=%d c0=%d n1=%d c1=%d makespan=%ld bound=%ld\n", P, n0, c0, n1,
                                   c1, (long)makespan, (long)bound);
                        }
                        ++cases;
                    }
    printf("%ld parameter sets, %ld failures\n", cases, bad);
    struct Shape {
        const char* name;
        int n0, c0, n1, c1;
    } xl[] = {{"qkv", 133, 131, 448, 41}, {"attn_proj", 147, 46, 448, 16}, {"fc", 175, 131, 448, 53},
              {"proj", 175, 131, 1600, 16}};
    for (const Shape& x : xl) {
        const GroupSched s{256, x.n0, x.c0, x.n1, x.c1};
        int64_t makespan = 0;
        for (int b = 0; b < 256; ++b) makespan = std::max(makespan, gs_finish(s, b));
        printf("%s: makespan %ld steps, ideal %ld\n", x.name, (long)makespan,
               (long)(((int64_t)x.n0 * x.c0 + (int64_t)x.n1 * x.c1 + 255) / 256));
    }
    return bad != 0;
}
