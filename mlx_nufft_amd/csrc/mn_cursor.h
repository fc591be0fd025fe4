// Key-range cursor shared by the owner-computes sweeps (mn_zsweep.hip,
// mn_ysweep.hip).
//
// A wavefront sweeps one block of grid columns along an axis. The points it
// takes at each step come from a few sources (its own block and the
// neighbour blocks whose footprints reach into it); with the sort key
// ordered (block, step, class), each (step, source) pair is one contiguous
// range of the sorted points. The cursor walks groups of ZG consecutive
// steps, NQ = ZG x sources ranges per group, and hands out batches of up to
// 64 consecutive elements of a group (in step-major order). Each lane finds
// its element's range by ballots of the range starts, so the cost does not
// grow with NQ.
//
// Memory waits on this target count outstanding loads in issue order, and
// the compiler can only wait for "all but the newest n" when every load is
// certain to have been issued. So the bounds of the next group are loaded
// one group ahead by every lane outside any branch (the fetch functor must
// do the same), and the usual single step to the next group is straight-
// line code: only a run of empty groups loops.
#pragma once

#include "mn_common.h"

namespace mn {

// The ranges of the current group, in LDS: element e of range q, with
// pf[q] <= e < pf[q + 1], is sorted point e + dj[q]; pf is the running sum
// of the range sizes.
template <int NQ>
struct __align__(16) SweepRanges {
    static_assert(NQ >= 1 && NQ <= 64, "at most one range per lane");
    int pf[NQ];
    int dj[NQ];
};

// The wave's position: the current group's first step zc, the next batch
// element and the group's element count (uniform), and the prefetched
// bounds [nst, nen) of range `lane` of group pzc.
struct SweepCursor {
    int zc, bat, tot;
    int pzc, nst, nen;
};

// fetch(zc, lane) returns (st, en): the sorted bounds of range `lane` of the
// group starting at step zc, (0, 0) for lanes >= NQ and absent ranges.
template <class Fetch>
__device__ __forceinline__ void sweep_fetch(SweepCursor &k, int zc, int lane, const Fetch fetch) {
    const int2 b = fetch(zc, lane);
    k.pzc = zc;
    k.nst = b.x;
    k.nen = b.y;
}

// Make group zc current (its ranges into rg) and start loading the bounds of
// the group after it.
template <int NQ, int ZG, class Fetch>
__device__ __forceinline__ void sweep_load(SweepCursor &k, int zc, SweepRanges<NQ> &rg, int lane,
                                           const Fetch fetch) {
    if (k.pzc != zc) sweep_fetch(k, zc, lane, fetch);
    const int st = k.nst, cnt = k.nen - k.nst;
    k.zc = zc;
    k.bat = 0;
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < NQ; d <<= 1) {
        const int v = __shfl_up(incl, d, 64);
        incl += (lane >= d) ? v : 0;
    }
    __syncthreads();  // earlier reads of rg are done
    if (lane < NQ) {
        rg.pf[lane] = incl - cnt;
        rg.dj[lane] = st - (incl - cnt);
    }
    k.tot = __shfl(incl, NQ - 1, 64);
    // the next group's bounds load only now, after this group's were used,
    // so using them never waits on the new loads
    sweep_fetch(k, zc + ZG, lane, fetch);
}

// Move past exhausted (or empty) groups; stops at zend.
template <int NQ, int ZG, class Fetch>
__device__ __forceinline__ void sweep_settle(SweepCursor &k, int zend, SweepRanges<NQ> &rg,
                                             int lane, const Fetch fetch) {
    if (k.bat >= k.tot && k.zc < zend) {
        sweep_load<NQ, ZG>(k, k.zc + ZG, rg, lane, fetch);
        while (k.bat >= k.tot && k.zc < zend) sweep_load<NQ, ZG>(k, k.zc + ZG, rg, lane, fetch);
    }
}

// One batch: its group's first step, its size (uniform; 0 when the sweep is
// done) and, per lane, whether the lane holds an element, its range index
// and its sorted index (0 for an idle lane, so loads indexed by it stay in
// bounds for P >= 1).
struct SweepBatch {
    int zc, nb;
    bool valid;
    int range;
    uint32_t j;
};

// Settle, then take the next batch. Lane j takes the last non-empty range
// that starts at a batch element in (0, j] (marked in qidx by element, so a
// ballot of the marks is a mask over elements), else the one holding the
// batch's first element.
template <int NQ, int ZG, class Fetch>
__device__ __forceinline__ SweepBatch sweep_next(SweepCursor &k, int zend, SweepRanges<NQ> &rg,
                                                 uint8_t *qidx, int lane, const Fetch fetch) {
    sweep_settle<NQ, ZG>(k, zend, rg, lane, fetch);
    SweepBatch s;
    s.zc = k.zc;
    s.nb = k.zc < zend ? min(64, k.tot - k.bat) : 0;
    s.valid = lane < s.nb;
    s.range = 0;
    s.j = 0;
    if (s.nb > 0) {
        __syncthreads();  // the ranges written by sweep_load are visible
        int d = 0;
        bool ne = false;
        if (lane < NQ) {
            const int st = rg.pf[lane];
            ne = (lane + 1 < NQ ? rg.pf[lane + 1] : k.tot) > st;
            d = st - k.bat;
        }
        // non-empty ranges starting at or before bat (ballot bit = range
        // index); the last holds bat (bat < tot, so there is one)
        const uint64_t mbefore = __ballot(ne && d <= 0);
        const int q0 = 63 - __clzll(mbefore);
        qidx[lane] = 0xff;
        __syncthreads();
        if (ne && d > 0 && d < 64) qidx[d] = (uint8_t)lane;
        __syncthreads();
        const uint64_t mpos = __ballot(qidx[lane] != 0xff);
        const uint64_t m = mpos & (lane == 63 ? ~0ull : ((2ull << lane) - 1));
        const int i = m ? (int)qidx[63 - __clzll(m)] : q0;
        const uint32_t jv = (uint32_t)(k.bat + lane + rg.dj[i]);
        s.range = i;
        s.j = s.valid ? jv : 0u;
    }
    if (k.zc < zend) k.bat += 64;
    return s;
}

}  // namespace mn
