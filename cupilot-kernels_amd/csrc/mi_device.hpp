// mi_device.hpp -- device-side helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi {

typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

// MI355X dispatches consecutive workgroups round-robin over its 8 XCDs, each
// with a private L2.  xcd_remap() turns the hardware order into an order in
// which every XCD receives one contiguous range of logical tile ids, so tiles
// that share A rows / B columns run on the same L2.  A bijection on [0, n).
constexpr int kNumXcd = 8;

__host__ __device__ __forceinline__ int xcd_remap(int bid, int n) {
    const int xcd = bid % kNumXcd;
    const int local = bid / kNumXcd;
    const int q = n / kNumXcd;
    const int r = n % kNumXcd;
    return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// Grouped raster: walk group_m tile-rows column by column so a wave of
// concurrently running tiles covers a compact block of C.
__host__ __device__ __forceinline__ void raster(int pid, int tiles_m, int tiles_n, int group_m,
                                                int& tm, int& tn) {
    const int in_group = group_m * tiles_n;
    const int g = pid / in_group;
    const int first_m = g * group_m;
    const int rows = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
    const int r = pid - g * in_group;
    tm = first_m + r % rows;
    tn = r / rows;
}

// Triangular tiling of an nt x nt tile grid.  The first nt(nt+1)/2 ids are
// the compute tiles, longest K range first: diagonal distance d = nt-1 down to
// 0, the distance-d band holding nt-d tiles that each reduce d+1 tiles of K.
// The remaining nt(nt-1)/2 ids are the off-structure tiles, row by row; the
// kernel writes them with zeros.  lower selects tril (tm >= tn) over triu.
// Returns false for an off-structure tile.
__host__ __device__ __forceinline__ bool tri_tile(int pid, int nt, bool lower, int& tm, int& tn) {
    const int ncomp = nt * (nt + 1) / 2;
    if (pid < ncomp) {
        int rem = pid, d = nt - 1;
        while (rem >= nt - d) {
            rem -= nt - d;
            --d;
        }
        tm = lower ? rem + d : rem;
        tn = lower ? rem : rem + d;
        return true;
    }
    int z = pid - ncomp, r = 0;
    while (z >= nt - 1 - r) {
        z -= nt - 1 - r;
        ++r;
    }
    tm = lower ? r : r + 1 + z;
    tn = lower ? r + 1 + z : r;
    return false;
}

// Chunked triangular work list (the 256-tile direct kernel).  Structure tile
// (tm, tn) reduces L = |tm - tn| + 1 tile-widths ("units") of K starting at
// unit min(tm, tn).  A tile longer than cap units is cut in two: its first
// cap units, written to C, and the rest, written to the mirror tile (tn, tm)
// -- which lies in the zero triangle, so C itself holds the partial sum until
// the finishing pass adds it in and zeroes the mirror.  Items run longest
// first, so workgroups dispatched in order as CUs free up balance the load:
// for l = cap, cap - 1, ..., 1 come (l == cap only) the first chunks of
// every long tile, longest tile first, then the second chunks of length l,
// then the whole tiles of length l (distance l - 1 from the diagonal).  At
// equal length a whole tile runs shorter -- the diagonal masks empty part
// of both its first and last unit, a chunk's only one of them -- so the
// list ends with the diagonal tiles (measured on 8192: 0.5-0.7 % faster
// than whole tiles before chunks).  Requires 2 cap >= nt (every second
// chunk is at most cap long).
__host__ __device__ __forceinline__ int tri_items(int nt, int cap) {
    const int nl = nt > cap ? nt - cap : 0;
    return nt * (nt + 1) / 2 + nl * (nl + 1) / 2;
}

// Item pid of that list: its tile, its K range [u0, u1) in units, and
// whether it goes to the mirror tile.
__host__ __device__ __forceinline__ void tri_item(int pid, int nt, int cap, bool lower, int& tm,
                                                  int& tn, int& u0, int& u1, int& mirror) {
    int rem = pid, d = 0, r = 0, first = 0, len = 0;
    mirror = 0;
    for (int l = cap; l >= 1; --l) {
        if (l == cap) {  // first chunks of the long tiles, L = nt down to cap + 1
            bool found = false;
            for (int L = nt; L > cap; --L) {
                if (rem < nt - L + 1) {
                    d = L - 1;
                    r = rem;
                    len = cap;
                    found = true;
                    break;
                }
                rem -= nt - L + 1;
            }
            if (found) break;
        }
        const int L = l + cap;  // second chunks of length l
        if (L <= nt) {
            if (rem < nt - L + 1) {
                d = L - 1;
                r = rem;
                first = cap;
                len = l;
                mirror = 1;
                break;
            }
            rem -= nt - L + 1;
        }
        if (rem < nt - (l - 1)) {  // whole tiles of length l
            d = l - 1;
            r = rem;
            len = l;
            break;
        }
        rem -= nt - (l - 1);
    }
    tm = lower ? r + d : r;
    tn = lower ? r : r + d;
    u0 = r + first;
    u1 = u0 + len;
}

// Zero-triangle tiles the chunked list's workgroups write with +0.0 once
// the compute items run out (dynamic order, cap >= 2): those at diagonal
// distance 1 .. cap - 1, i.e. every zero tile except the mirror tiles
// (distance >= cap, which park second-chunk partials for the finishing pass)
// and the tile holding the item counter ((0, 1) lower, (1, 0) upper, which
// the finishing pass zeroes).  Item z of them, by distance, then row.
__host__ __device__ __forceinline__ int tri_zero_items(int nt, int cap) {
    if (cap < 2 || nt < 2) return 0;
    const int dmax = cap - 1 < nt - 1 ? cap - 1 : nt - 1;
    return dmax * nt - dmax * (dmax + 1) / 2 - 1;
}
__host__ __device__ __forceinline__ void tri_zero_tile(int z, int nt, bool lower, int& tm, int& tn) {
    int rem = z + 1, d = 1;  // + 1: skip the counter tile, distance 1 row 0
    while (rem >= nt - d) {
        rem -= nt - d;
        ++d;
    }
    tm = lower ? rem : rem + d;
    tn = lower ? rem + d : rem;
}

// Stream-K schedule (dense products on a persistent grid of G workgroups).
// The T output tiles of one product, in raster order, are split into n_dp
// data-parallel tiles (a multiple of G: whole waves, each tile reduced by one
// workgroup) followed by S = T - n_dp stream-K tiles, whose S * ipt K-slices
// (ipt slices per tile) are dealt out as G contiguous, equal ranges:
// logical workgroup lg (= xcd_remap of its hardware index, so the ranges of
// one XCD are neighbours in the raster) takes slices
// [sk_begin(lg), sk_begin(lg + 1)).  A range may start inside a tile only
// once, at its first slice, so every workgroup produces at most one partial
// tile that does not start at k = 0: it goes to workspace slot lg; every
// segment that starts at k = 0 (a whole tile, or the head of a split one) is
// written to C.  sk_fixup then adds the slots of each split tile into C in
// increasing lg order (increasing k): a fixed order, so results are
// deterministic.  Slices are indexed with 64-bit integers (S * ipt * G can
// pass 2^31).
__host__ __device__ __forceinline__ int64_t sk_begin(int64_t lg, int64_t iters, int G) {
    return lg * iters / G;
}

// Logical workgroup whose range holds slice x (the largest lg with
// sk_begin(lg) <= x).
__host__ __device__ __forceinline__ int64_t sk_owner(int64_t x, int64_t iters, int G) {
    return ((x + 1) * G - 1) / iters;
}

// Work item `item` of hardware workgroup b: first its n_dp / G data-parallel
// tiles (walk index b + i G, placed by xcd_remap over n_dp), then the
// segments of its stream-K range, one per tile it touches.  Returns false
// past its last item; else the logical tile index lt (raster position), the
// slice range [s0, s1) within that tile and whether the partial goes to the
// workspace (slot = logical workgroup).
__host__ __device__ __forceinline__ bool sk_work(int b, int item, int G, int n_dp, int64_t S,
                                                 int ipt, int& lt, int& s0, int& s1, int& to_ws) {
    const int dp_items = n_dp / G;
    if (item < dp_items) {
        lt = xcd_remap(b + item * G, n_dp);
        s0 = 0;
        s1 = ipt;
        to_ws = 0;
        return true;
    }
    const int j = item - dp_items;
    const int64_t iters = S * ipt;
    const int lg = xcd_remap(b, G);
    const int64_t beg = sk_begin(lg, iters, G), end = sk_begin(lg + 1, iters, G);
    int64_t x;
    if (beg % ipt == 0) {
        x = beg + (int64_t)j * ipt;
    } else {
        x = j == 0 ? beg : (beg / ipt + 1) * ipt + (int64_t)(j - 1) * ipt;
    }
    if (x >= end) return false;
    const int64_t t = x / ipt;
    const int64_t xe = end < (t + 1) * ipt ? end : (t + 1) * ipt;
    lt = n_dp + (int)t;
    s0 = (int)(x - t * ipt);
    s1 = (int)(xe - t * ipt);
    to_ws = s0 != 0;
    return true;
}

// Workspace slots holding the partials of stream-K tile t (0 <= t < S), in
// the order they are added: [first, first + count), count 0 when one
// workgroup reduced the whole tile.
__host__ __device__ __forceinline__ void sk_fixup_slots(int64_t t, int64_t S, int ipt, int G,
                                                        int64_t& first, int64_t& count) {
    const int64_t iters = S * ipt;
    const int64_t head = sk_owner(t * ipt, iters, G);
    const int64_t last = sk_owner((t + 1) * ipt - 1, iters, G);
    first = head + 1;
    count = last - head;
}

// Phased stream-K.  With the contiguous ranges above every workgroup starts
// at its own K offset, so the workgroups that run together on one XCD read
// unrelated slices and share nothing in L2 (3072^2 x 8192 on the 256 tile:
// 11 % L2 hits, 10x the compulsory bytes fetched).  The phased schedule deals
// the same S x ipt slices out so that, at any moment, the workgroups of one
// XCD read the same K-slice of neighbouring tiles.  Each logical workgroup
// has a budget of B slice-times, and a segment costs its slices plus kSkSegCost
// (the store of its partial tile and the restart of the pipeline).  Charging
// nothing for segments gave some workgroups a third one and ran 0.2-1 %
// slower than the ranges; 1 slice, 0.3 % slower on 4608^3 and 1 % on 3584^3
// (11 phases); 2 slices with at most 8 phases, against the ranges in one
// process (10 shapes, medians of 3): 0.978-0.999 of their time on 7
// (1536^2 x 4096 0.978, 3328^2 x 4096 0.983, 3072^2 x 8192 0.994-0.996),
// 1.000-1.001 on 4352^3 and 4608^3, 1.005 on 3584^3.  A
// phase serves n tiles t0 .. t0 + n - 1 with the n logical workgroups
// w0 .. w0 + n - 1 (workgroup w0 + i takes tile t0 + i), every one of them
// reducing the same K range [k0, k1) and starting it at the same moment:
//   * n_t tiles left (each needing [k_lo, ipt), r = ipt - k_lo slices),
//     n_w workgroups left (each with budget c left);
//   * n_t <= n_w: the first n_t workgroups reduce [k_lo, k_lo + min(c - cost,
//     r)) of every tile and are used up; if that was all of r, the schedule
//     is complete;
//   * n_t > n_w: every workgroup reduces the whole rest [k_lo, ipt) of one
//     tile and keeps c - r - cost for the next phase.
// All workgroups in a phase have run the same earlier phases, so their
// segments start together; consecutive logical workgroups (one XCD's, via
// xcd_remap) take consecutive tiles of the raster, which share A row and B
// column panels.  A segment that starts at k = 0 is written to C; every
// other segment to its own workspace slot, slots numbered tile by tile in k
// order, so the fixup adds a tile's slots [first, first + count) in order --
// deterministic.  The planner takes the smallest budget the phases can meet
// within kSkMaxPhases entries and kSkMaxSegments segments per workgroup, and
// uses the phases only where that budget is no more than the busiest
// workgroup's cost under the contiguous ranges (sk_ranges_cost); otherwise
// the ranges (nph = 0).  Example, 3072^2 x 8192 on the 256 tile (S = 144
// tiles of ipt = 256 slices, G = 256): tiles 0..143 reduce [0, 145) on
// workgroups 0..143; tiles 0..111 [145, 256) on 144..255; tiles 112..143
// [145, 177), [177, 209), [209, 241) on 144..175, 176..207, 208..239; then
// [241, 256) on 240..255 for tiles 112..127 and again for 128..143.
constexpr int kSkMaxPhases = 8;
constexpr int kSkMaxSegments = 3;
constexpr int kSkSegCost = 2;
struct SkPhase {
    int t0, n, k0, k1, w0;
};

// Host: the phase table of S tiles x ipt slices over G workgroups with a
// budget of B slice-times each.  Returns the most segments any workgroup
// gets, or -1 where the budget is too small or the table would not fit
// kSkMaxPhases; slots = the segments that do not start at k = 0.
inline int sk_build_phases(int64_t S, int64_t ipt, int64_t G, int64_t B, SkPhase* ph, int& nph,
                           int64_t& slots) {
    nph = 0;
    slots = 0;
    if (S <= 0 || ipt <= 0 || G <= 0 || S > G) return -1;
    int64_t c = B;
    int64_t t_lo = 0, k_lo = 0, w_lo = 0;
    int t2 = 0, most = 0;  // whole-rest phases so far; most segments of a used-up workgroup
    for (;;) {
        const int64_t n_t = S - t_lo, r = ipt - k_lo, n_w = G - w_lo;
        if (n_t == 0) break;
        if (nph == kSkMaxPhases || n_w <= 0) return -1;
        if (n_t <= n_w) {
            const int64_t len = c - kSkSegCost < r ? c - kSkSegCost : r;
            if (len <= 0) return -1;
            ph[nph++] = SkPhase{(int)t_lo, (int)n_t, (int)k_lo, (int)(k_lo + len), (int)w_lo};
            if (k_lo > 0) slots += n_t;
            most = most > t2 + 1 ? most : t2 + 1;
            if (len == r) break;
            k_lo += len;
            w_lo += n_t;
        } else {
            if (r + kSkSegCost > c) return -1;
            ph[nph++] = SkPhase{(int)t_lo, (int)n_w, (int)k_lo, (int)ipt, (int)w_lo};
            if (k_lo > 0) slots += n_w;
            ++t2;
            t_lo += n_w;
            c -= r + kSkSegCost;
        }
    }
    return most > t2 ? most : t2;
}

// Host: the busiest workgroup's cost (slices + kSkSegCost per segment) under
// the contiguous ranges.
// (The planner asks this for every candidate tile config, so it walks the
// ranges incrementally: range lg is [lg I / G, (lg + 1) I / G) with
// I = S ipt, and its first and last slices' tiles only move forward.)
inline int64_t sk_ranges_cost(int64_t S, int64_t ipt, int64_t G) {
    const int64_t iters = S * ipt, q = iters / G, rem = iters % G;
    int64_t most = 0, b = 0, acc = 0, tb = 0, te = 0;  // tb = b / ipt, te = (e - 1) / ipt
    for (int64_t lg = 0; lg < G; ++lg) {
        int64_t e = b + q;
        acc += rem;
        if (acc >= G) {
            acc -= G;
            ++e;
        }
        if (e > b) {
            while ((tb + 1) * ipt <= b) ++tb;
            while ((te + 1) * ipt <= e - 1) ++te;
            const int64_t cost = e - b + kSkSegCost * (te - tb + 1);
            most = cost > most ? cost : most;
        }
        b = e;
    }
    return most;
}

// Slot numbering of the phased schedule: the slots of tile t start after
// those of tiles 0 .. t - 1; nph entries of ph.
__host__ __device__ __forceinline__ int64_t sk_ph_first_slot(int64_t t, const SkPhase* ph, int nph) {
    int64_t first = 0;
    for (int q = 0; q < nph; ++q) {
        if (ph[q].k0 == 0) continue;
        const int64_t d = t - ph[q].t0;
        first += d <= 0 ? 0 : d < ph[q].n ? d : ph[q].n;
    }
    return first;
}

// Phased schedule, the item-th segment (in run order) of logical workgroup
// lg: tile t (0-based among the stream-K tiles), slice range [s0, s1), and
// its slot (-1: the segment starts at k = 0 and goes to C).
__host__ __device__ __forceinline__ bool sk_ph_work(int lg, int item, const SkPhase* ph, int nph,
                                                    int64_t& t, int& s0, int& s1, int64_t& slot) {
    int seen = 0;
    for (int q = 0; q < nph; ++q) {
        if (lg < ph[q].w0 || lg >= ph[q].w0 + ph[q].n) continue;
        if (seen++ != item) continue;
        t = ph[q].t0 + (lg - ph[q].w0);
        s0 = ph[q].k0;
        s1 = ph[q].k1;
        if (s0 == 0) {
            slot = -1;
            return true;
        }
        int64_t before = 0;  // earlier phases that parked a part of tile t
        for (int e = 0; e < q; ++e)
            if (ph[e].k0 > 0 && t >= ph[e].t0 && t < ph[e].t0 + ph[e].n) ++before;
        slot = sk_ph_first_slot(t, ph, nph) + before;
        return true;
    }
    return false;
}

// Phased schedule: the slots of stream-K tile t, [first, first + count).
__host__ __device__ __forceinline__ void sk_ph_fixup_slots(int64_t t, const SkPhase* ph, int nph,
                                                           int64_t& first, int64_t& count) {
    first = sk_ph_first_slot(t, ph, nph);
    count = 0;
    for (int q = 0; q < nph; ++q)
        if (ph[q].k0 > 0 && t >= ph[q].t0 && t < ph[q].t0 + ph[q].n) ++count;
}

// Either schedule (nph = 0: contiguous ranges, else the phase table): work
// item `item` of hardware workgroup b -- its n_dp / G data-parallel tiles,
// then its stream-K segments.  lt = the tile's raster position, [s0, s1) its
// slices, slot = the workspace slot of a segment that does not start at
// k = 0, else -1 (written to C).
__host__ __device__ __forceinline__ bool sk_item(int b, int item, int G, int n_dp, int64_t S,
                                                 int ipt, const SkPhase* ph, int nph, int& lt,
                                                 int& s0, int& s1, int64_t& slot) {
    if (nph == 0 || item < n_dp / G) {
        int to_ws;
        if (!sk_work(b, item, G, n_dp, S, ipt, lt, s0, s1, to_ws)) return false;
        slot = to_ws ? xcd_remap(b, G) : -1;
        return true;
    }
    int64_t t;
    if (!sk_ph_work(xcd_remap(b, G), item - n_dp / G, ph, nph, t, s0, s1, slot)) return false;
    lt = n_dp + (int)t;
    return true;
}

// Either schedule: the slots the fixup adds into stream-K tile t, in order.
// Contiguous ranges leave a slot empty where its workgroup got no slices
// (sk_slot_used); the phase table never does.
__host__ __device__ __forceinline__ void sk_tile_slots(int64_t t, int64_t S, int ipt, int G,
                                                       const SkPhase* ph, int nph, int64_t& first,
                                                       int64_t& count) {
    if (nph == 0)
        sk_fixup_slots(t, S, ipt, G, first, count);
    else
        sk_ph_fixup_slots(t, ph, nph, first, count);
}
__host__ __device__ __forceinline__ bool sk_slot_used(int64_t slot, int64_t S, int ipt, int G, int nph) {
    const int64_t iters = S * ipt;
    return nph > 0 || sk_begin(slot + 1, iters, G) != sk_begin(slot, iters, G);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    uint64_t z = x + 0x9E3779B97F4A7C15ULL;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float uniform_from_bits(uint64_t z) {
    return (float)(uint32_t)(z >> 40) * 0x1p-23f - 1.0f;
}

}  // namespace mi
