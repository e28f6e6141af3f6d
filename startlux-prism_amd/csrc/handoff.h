// Balanced-grid decode kernels (the Q8_0 and Q4_K "stream" kernels): the walk of a workgroup's equal share of a
// projection's (16-row weight tile, unit) sequence, the handoff of running fp32 sums between neighbouring workgroups
// through a zeroed workspace, and the LDS counters their compute and fold waves meet at.
//
// A projection's work is tiles x KP units (a unit: the 64 inputs of a Q8_0 block pair, the 256 of a Q4_K
// super-block).  W workgroups take ranges of total / W or one more units, so a range starts and ends inside tiles:
// its first tile's units continue a tile whose first units belong to the previous workgroup (a "tail"), its last
// tile's units start a tile the next workgroup finishes (a "head").  Every output's fp32 sum over units runs in unit
// order, so a tail's fold starts from the head's running sums.  A workgroup walks its tiles last to first: the head
// first (its running sums handed on as soon as they are complete), whole tiles in between, the tail last (by when
// the previous workgroup has long published its head).  A round is up to RP units of one tile.
//
// Handoff protocol (per output word, never leaves a word set after a launch that completes): each launch carries a
// tag (hand_next_tag: 1 .. 2^32 - 2, a different one per launch made by the library); the producer writes
// tag << 32 | bits with a compare-and-swap from 0 (whose result it checks at its end); the consumer takes the bits
// only under its own launch's tag, normally read one round ahead, else by polling, and clears the word.  A consumer
// that polls past its bound (a predecessor that never ran: not expected, every predecessor is dispatched first and
// publishes before it waits on anything) swaps in the "abandoned" tag and takes its value if the producer had just
// finished, or yields NaN outputs (loud, never silently wrong); a producer that finds "abandoned" clears the word.  A
// word left set by an earlier launch that did not complete (killed, or two streams overlapping on one workspace)
// carries another tag: the consumer never takes it, and the producer whose compare-and-swap it defeated replaces it
// with its own value at its end.  What is not detected: a stale word under the same tag, which only a captured
// graph replayed after a replay of it was killed can leave (a captured launch keeps the tag it was recorded with).
#pragma once

#include <atomic>

#include "common.h"

namespace prism {

constexpr unsigned kTagAbandoned = 0xffffffffu;

// The next launch's tag (host side): never 0 (an empty word) nor kTagAbandoned.
inline unsigned hand_next_tag() {
    static std::atomic<unsigned> counter{0};
    return counter.fetch_add(1, std::memory_order_relaxed) % 0xfffffffeu + 1u;
}

__device__ __forceinline__ unsigned long long hand_load(unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void hand_store(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Takes the previous workgroup's y published under `tag` (bounded wait).
__device__ __forceinline__ float hand_take(unsigned long long* p, unsigned tag) {
    for (int it = 0; it < (1 << 22); it++) {
        const unsigned long long v = hand_load(p);
        if ((v >> 32) == tag) {
            hand_store(p, 0);
            return __uint_as_float((uint32_t)v);
        }
        __builtin_amdgcn_s_sleep(2);
    }
    const unsigned long long old =
        __hip_atomic_exchange(p, (unsigned long long)kTagAbandoned << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((old >> 32) == tag) {
        hand_store(p, 0);
        return __uint_as_float((uint32_t)old);
    }
    return __uint_as_float(0x7fc00000u);
}

__device__ __forceinline__ unsigned long long hand_word(float y, unsigned tag) {
    return (unsigned long long)tag << 32 | __float_as_uint(y);
}

// Publishes `word` without waiting for the compare-and-swap's result (returned, for hand_settle at the end).
__device__ __forceinline__ unsigned long long hand_publish(unsigned long long* p, unsigned long long word) {
    unsigned long long expect = 0;
    __hip_atomic_compare_exchange_strong(p, &expect, word, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return expect;
}

// The producer's check at its end, `old` being hand_publish's result: 0, the publish stood; "abandoned", the
// consumer gave up (clear the word); anything else is a stale word of another launch that the publish did not
// replace: replace it now (the consumer polls for this launch's tag meanwhile, or abandons it).
__device__ __forceinline__ void hand_settle(unsigned long long* p, unsigned long long old, unsigned long long word) {
    for (int it = 0; it < 4 && old != 0; it++) {
        if ((old >> 32) == kTagAbandoned) {
            hand_store(p, 0);
            return;
        }
        unsigned long long expect = old;
        if (__hip_atomic_compare_exchange_strong(p, &expect, word, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT))
            return;
        old = expect;
    }
}

// Bounded wait on an LDS counter (workgroup scope): every wave of the workgroup is resident, so the counter's
// producers always progress; the bound only keeps a broken launch from spinning forever.
__device__ __forceinline__ void lds_wait_ge(unsigned* c, unsigned target) {
    for (int it = 0; it < (1 << 24); it++) {
        if (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
        __builtin_amdgcn_s_sleep(1);
    }
}

// One round of a workgroup's walk: tile nt, units p0 .. p0 + np - 1 of it; `first` / `last`: the round opens /
// closes a fragment (the tile's part inside this workgroup's range), whose units are ps .. pe - 1.
struct Round {
    int nt, p0, np, ps, pe;
    bool first, last;
};

// Workgroup v of W over `tiles` tiles of KP units, rounds of RP units (tiles * KP < 2^31: 32-bit arithmetic).
struct Walk {
    int KP, RP, RT, nt_lo, nt_hi, ps_lo, ps_hi, pe_hi, r_hi, nmid, r_lo, NR;
    __device__ __forceinline__ Walk(int tiles, int kp, int rp, int W, int v) : KP(kp), RP(rp) {
        const int total = tiles * KP;
        const int cq = total / W, cr = total - cq * W;
        const int c0 = v * cq + min(v, cr), c1 = c0 + cq + (v < cr ? 1 : 0);
        nt_lo = c0 / KP;
        nt_hi = (c1 - 1) / KP;
        ps_lo = c0 - nt_lo * KP;
        pe_hi = c1 - nt_hi * KP;
        RT = (KP + RP - 1) / RP;
        ps_hi = nt_hi == nt_lo ? ps_lo : 0;
        r_hi = (pe_hi - ps_hi + RP - 1) / RP;
        nmid = max(0, nt_hi - nt_lo - 1);
        r_lo = nt_lo < nt_hi ? (KP - ps_lo + RP - 1) / RP : 0;
        NR = r_hi + nmid * RT + r_lo;
    }
    __device__ __forceinline__ Round round(int rho) const {
        Round d;
        int lr;
        if (rho < r_hi) {
            d.nt = nt_hi, d.ps = ps_hi, d.pe = pe_hi, lr = rho;
        } else if (rho - r_hi < nmid * RT) {
            const int x = rho - r_hi;
            d.nt = nt_hi - 1 - x / RT, d.ps = 0, d.pe = KP, lr = x % RT;
        } else {
            d.nt = nt_lo, d.ps = ps_lo, d.pe = KP, lr = rho - r_hi - nmid * RT;
        }
        d.p0 = d.ps + lr * RP;
        d.np = max(0, min(RP, d.pe - d.p0));
        d.first = lr == 0;
        d.last = d.p0 + RP >= d.pe;
        if (rho >= NR) d.np = 0, d.first = d.last = false;     // prefetch past the end: clamped, unused
        return d;
    }
};

}  // namespace prism
