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
