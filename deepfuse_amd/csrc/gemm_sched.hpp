// gemm_sched.hpp -- static schedule of the grouped backward launch: one
// persistent grid runs the work units of two GEMMs, the dW units first
// (few, long: up to 128 K steps each) and the dX units after them (many,
// short), so the CUs that get no dW unit start on dX at once instead of
// idling until dW is done.
//
// Units of problem 0 (n0 of them, cost c0 each) go round-robin to the P
// logical blocks: block b gets d0(b) of them and becomes free at
// f(b) = d0(b) * c0.  The units of problem 1 (n1, cost c1 each) are then
// dealt in time order: block b would start its k-th one at f(b) + k * c1,
// and the unit it gets is the rank of that start event among all blocks'
// events (earlier time first, lower block first on a tie).  Blocks free at
// the same time therefore take neighbouring units, which keeps the tiles
// running together on one XCD adjacent in the tile order.
//
// f(b) takes two values: blocks b < nA hold one unit more than the rest.
// Ranks are counted in closed form per class, so a block finds its k-th
// unit in O(1) and its unit count in O(units) -- no tables, no atomics.
// Every function here is plain integer arithmetic shared by the host
// (planning, tests) and the device (the kernel's unit walk).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define DF_HD __host__ __device__ __forceinline__
#else
#define DF_HD inline
#endif

namespace dfk {

struct GroupSched {
    int P;       // logical blocks
    int n0, c0;  // problem-0 units and their cost (steps)
    int n1, c1;  // problem-1 units and their cost (steps), c1 >= 1
};

// problem-0 units of block b (round-robin)
DF_HD int gs_d0(const GroupSched& s, int b) { return b < s.n0 ? (s.n0 - b + s.P - 1) / s.P : 0; }

// events k >= 0 of a class free at f with f + k*c1 < t
DF_HD int64_t gs_before(int64_t t, int64_t f, int64_t c1) { return t > f ? (t - f - 1) / c1 + 1 : 0; }

// rank of block b's k-th problem-1 start among all blocks' start events
DF_HD int64_t gs_rank(const GroupSched& s, int b, int k) {
    const int lo = s.n0 / s.P;
    const int nA = s.n0 - lo * s.P;  // blocks holding lo + 1 problem-0 units
    const int64_t fA = (int64_t)(lo + 1) * s.c0, fB = (int64_t)lo * s.c0;
    const bool inA = b < nA;
    const int64_t t = (inA ? fA : fB) + (int64_t)k * s.c1;
    int64_t r = (int64_t)nA * gs_before(t, fA, s.c1) + (int64_t)(s.P - nA) * gs_before(t, fB, s.c1);
    // ties at time t, lower blocks first
    if (t >= fA && (t - fA) % s.c1 == 0) r += inA ? b : nA;
    if (!inA && t >= fB && (t - fB) % s.c1 == 0) r += b - nA;
    return r;
}

// problem-1 units of block b: ranks grow with k, so count until one lands
// past the last unit
DF_HD int gs_d1(const GroupSched& s, int b) {
    int k = 0;
    while (gs_rank(s, b, k) < s.n1) ++k;
    return k;
}

// block b's r-th unit: (problem, unit index within that problem)
DF_HD void gs_unit(const GroupSched& s, int b, int r, int& prob, int& unit) {
    const int d0 = gs_d0(s, b);
    if (r < d0) {
        prob = 0;
        unit = b + r * s.P;
    } else {
        prob = 1;
        unit = (int)gs_rank(s, b, r - d0);
    }
}

// finishing time of block b (the schedule's makespan is the max over b)
DF_HD int64_t gs_finish(const GroupSched& s, int b) {
    return (int64_t)gs_d0(s, b) * s.c0 + (int64_t)gs_d1(s, b) * s.c1;
}

}  // namespace dfk
