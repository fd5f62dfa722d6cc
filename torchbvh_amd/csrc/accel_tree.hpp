// Radix-tree (Karras 2012) helpers shared by the accel kernels and the
// fused first tree pass: the sorted-code view, the node search, the exact
// box of a sorted range from an implicit tree (global or LDS-resident) and
// the child reference encoding.
#pragma once

#include <float.h>

#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

// Sorted codes of one cloud, read from an LDS window where it covers the
// position and from global memory elsewhere.
struct CodeView {
    const uint32_t* codes;  // cloud's codes (global)
    const uint32_t* win;    // LDS window, cloud-local positions [w_lo, w_hi)
    int w_lo, w_hi;
    int n;
    __device__ __forceinline__ uint32_t at(int j) const {
        return (j >= w_lo && j < w_hi) ? win[j - w_lo] : codes[j];
    }
    // Length of the common prefix of the 64-bit keys (code << 32 | position)
    // at positions i and j; -1 outside the cloud.
    __device__ __forceinline__ int prefix_len(int i, uint32_t ci, int j) const {
        if (j < 0 || j >= n) return -1;
        const uint64_t a = (static_cast<uint64_t>(ci) << 32) | static_cast<uint32_t>(i);
        const uint64_t b = (static_cast<uint64_t>(at(j)) << 32) | static_cast<uint32_t>(j);
        return __clzll(static_cast<long long>(a ^ b));
    }
};

template <int D>
__device__ __forceinline__ void merge_row(float* box, const float* row) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
        box[d] = fminf(box[d], row[d]);
        box[D + d] = fmaxf(box[D + d], row[D + d]);
    }
}

// Exact box of sorted positions [a, b] (inclusive) from the implicit tree:
// heap node h has 1-based index h + 1, leaves are [2^L, 2^(L+1)), and the
// classic bottom-up cover visits O(log n) nodes whose ranges tile [a, b].
template <int D>
__device__ void range_box(const float* nodes, int vl, int L, int a, int b, float* box) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
        box[d] = FLT_MAX;
        box[D + d] = -FLT_MAX;
    }
    int64_t lo = static_cast<int64_t>(a) + (int64_t(1) << L);
    int64_t hi = static_cast<int64_t>(b) + 1 + (int64_t(1) << L);
    // The cover rows of the next kLevels levels follow from lo and hi
    // alone: all are loaded before any is merged (one memory round trip per
    // kLevels levels instead of per level), then merged in level order.
    constexpr int kLevels = 4;
    while (lo < hi) {
        float rl[kLevels][2 * D], rh[kLevels][2 * D];
        bool tl[kLevels], th[kLevels];
#pragma unroll
        for (int u = 0; u < kLevels; ++u) {
            const bool live = lo < hi;
            tl[u] = live && (lo & 1);
            if (tl[u]) {
                const float* row = nodes + static_cast<int64_t>(tree::memory_index(vl, L, static_cast<int>(lo - 1))) * 2 * D;
#pragma unroll
                for (int c = 0; c < 2 * D; ++c) rl[u][c] = row[c];
                ++lo;
            }
            th[u] = live && (hi & 1);
            if (th[u]) {
                --hi;
                const float* row = nodes + static_cast<int64_t>(tree::memory_index(vl, L, static_cast<int>(hi - 1))) * 2 * D;
#pragma unroll
                for (int c = 0; c < 2 * D; ++c) rh[u][c] = row[c];
            }
            if (live) {
                lo >>= 1;
                hi >>= 1;
            }
        }
#pragma unroll
        for (int u = 0; u < kLevels; ++u) {
            if (tl[u]) merge_row<D>(box, rl[u]);
            if (th[u]) merge_row<D>(box, rh[u]);
        }
    }
}

// range_box over a work-group's LDS copy of an implicit subtree: a 0-based
// heap of `width` leaves (node k's children 2k + 1, 2k + 2), [a, b] in
// group-local leaf positions.  The same node sequence and merge order as
// range_box, so the boxes are bit-identical.
template <int D>
__device__ void range_box_lds(const float* s_box, int width, int a, int b, float* box) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
        box[d] = FLT_MAX;
        box[D + d] = -FLT_MAX;
    }
    int lo = a + width;
    int hi = b + 1 + width;
    while (lo < hi) {
        if (lo & 1) {
            merge_row<D>(box, s_box + (lo - 1) * 2 * D);
            ++lo;
        }
        if (hi & 1) {
            --hi;
            merge_row<D>(box, s_box + (hi - 1) * 2 * D);
        }
        lo >>= 1;
        hi >>= 1;
    }
}

// Positions of sorted codes kept in LDS on each side of a work-group's own.
constexpr int kCodeHalo = 256;

// Direction of radix-tree node i (Karras 2012, section 4: towards the
// neighbour with the longer common prefix) and the prefix length its range
// must exceed.
__device__ __forceinline__ void karras_dir(const CodeView& cv, int i, uint32_t ci, int& dir, int& dmin) {
    dir = cv.prefix_len(i, ci, i + 1) - cv.prefix_len(i, ci, i - 1) > 0 ? 1 : -1;
    dmin = cv.prefix_len(i, ci, i - dir);
}

// Range [first, last] and split gamma of node i (the left child covers
// [first, gamma], the right [gamma + 1, last]) given its direction, with
// `lmax` a power of two greater than the range's extent from i.
__device__ __forceinline__ void karras_range(const CodeView& cv, int i, uint32_t ci, int dir, int dmin, int lmax,
                                             int& first, int& last, int& gamma) {
    int l = 0;
    for (int t = lmax >> 1; t >= 1; t >>= 1) {
        if (cv.prefix_len(i, ci, i + (l + t) * dir) > dmin) l += t;
    }
    const int j = i + l * dir;
    const int dnode = cv.prefix_len(i, ci, j);
    int split = 0;
    int t = l;
    do {
        t = (t + 1) >> 1;
        if (cv.prefix_len(i, ci, i + (split + t) * dir) > dnode) split += t;
    } while (t > 1);
    gamma = i + split * dir + (dir < 0 ? dir : 0);
    first = min(i, j);
    last = max(i, j);
}

// Node i of a cloud's radix tree: direction, exponential search for the
// range's extent, then karras_range.
__device__ __forceinline__ void karras_node(const CodeView& cv, int i, int& first, int& last, int& gamma) {
    const uint32_t ci = cv.at(i);
    int dir, dmin;
    karras_dir(cv, i, ci, dir, dmin);
    int lmax = 2;
    while (cv.prefix_len(i, ci, i + lmax * dir) > dmin) lmax <<= 1;
    karras_range(cv, i, ci, dir, dmin, lmax, first, last, gamma);
}

// Both child boxes of a record, as D 16-byte stores (record rows are 64 B
// in 3-D and 48 B in 2-D from a 256-byte aligned base, so every row is
// 16-byte aligned); one lane's row in one instruction per 16 bytes instead
// of one per float.
template <int D>
__device__ __forceinline__ void store_boxes(float* rec, const float* lbox, const float* rbox) {
    float v[4 * D];
#pragma unroll
    for (int c = 0; c < 2 * D; ++c) {
        v[c] = lbox[c];
        v[2 * D + c] = rbox[c];
    }
    float4* r4 = reinterpret_cast<float4*>(rec);
#pragma unroll
    for (int u = 0; u < D; ++u) r4[u] = make_float4(v[4 * u], v[4 * u + 1], v[4 * u + 2], v[4 * u + 3]);
}

template <int D>
__device__ __forceinline__ int32_t child_ref(int first, int last, int internal) {
    const int count = last - first + 1;
    if (count <= accel_bucket<D>()) {
        return static_cast<int32_t>(0x80000000u | (static_cast<uint32_t>(count - 1) << 28) |
                                    static_cast<uint32_t>(first));
    }
    return internal;
}

// Child refs and parent links of radix-tree node i with range [first, last]
// and split gamma (`records`: the cloud's first record row).  The node
// writes its own child refs and its children's parent links: word 4D + 2
// of an internal child's row, word 4D + 3 of the row where a bucket child
// starts; the root also writes its own parent word (-1).  Every word has
// exactly one writer, so no ordering between nodes is needed.
template <int D>
__device__ __forceinline__ void link_record(float* records, int i, int first, int gamma, int last) {
    constexpr int R = 4 * D + 4;
    float* rec = records + static_cast<int64_t>(i) * R;
    const int32_t lref = child_ref<D>(first, gamma, gamma);
    const int32_t rref = child_ref<D>(gamma + 1, last, gamma + 1);
    *reinterpret_cast<float2*>(rec + 4 * D) = make_float2(__int_as_float(lref), __int_as_float(rref));
    if (i == 0) rec[4 * D + 2] = __int_as_float(-1);
    records[static_cast<int64_t>(lref >= 0 ? lref : first) * R + 4 * D + (lref >= 0 ? 2 : 3)] = __int_as_float(i);
    records[static_cast<int64_t>(rref >= 0 ? rref : gamma + 1) * R + 4 * D + (rref >= 0 ? 2 : 3)] =
        __int_as_float(i);
}

}  // namespace
}  // namespace tbvh
