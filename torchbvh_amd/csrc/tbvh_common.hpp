// Shared host/device definitions: implicit-tree closed forms, Morton
// quantisation and the segment descriptor used by every kernel.
//
// The implicit tree is the "ostensibly implicit" layout used by the reference
// (torchbvh/csrc/implicit_tree.cuh:21-127): a complete binary tree in heap
// order over 2^L leaf slots (L = ceil(log2 n)); the last 2^L - n leaf slots are
// virtual, an internal node is virtual iff both children are, and only real
// nodes are stored, level by level.  Because the virtual nodes of every level
// form a suffix of that level, a real node's storage row is its heap index
// minus the number of virtual nodes on the levels above it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define TBVH_HD __host__ __device__ __forceinline__

namespace tbvh {

// ---------------------------------------------------------------------------
// Implicit-tree closed forms (reference: implicit_tree.cuh:26-127)
// ---------------------------------------------------------------------------
namespace tree {

TBVH_HD int floor_log2(uint32_t x) { return 31 - __builtin_clz(x); }

// ceil(log2 x) with ceil_log2(0) = ceil_log2(1) = 0.
TBVH_HD int ceil_log2(uint32_t x) { return x <= 1u ? 0 : floor_log2(x - 1u) + 1; }

TBVH_HD int popcount(uint32_t x) { return __builtin_popcount(x); }

// Level holding the leaves of a tree over n points.
TBVH_HD int leaf_level(int n) { return ceil_log2(static_cast<uint32_t>(n)); }

// Number of virtual leaf slots at the leaf level.
TBVH_HD int virtual_leaves(int n) { return (1 << leaf_level(n)) - n; }

// Real nodes: n leaves + (n - 1) internal nodes with two children, plus one
// internal node with a single real child for every level whose count of
// virtual nodes is odd, i.e. one per set bit of the virtual-leaf count.
// For n <= 2^30 the count fits in int (2^31 - 1 at n = 2^30, where the
// popcount is 0); n + (n - 1) keeps the partial sums in range too, where
// 2 * n would overflow at n = 2^30.
TBVH_HD int real_node_count(int n) {
    return n + (n - 1) + popcount(static_cast<uint32_t>(virtual_leaves(n)));
}

TBVH_HD int level_of(int i) { return floor_log2(static_cast<uint32_t>(i) + 1u); }
TBVH_HD int level_first(int level) { return (1 << level) - 1; }

// Virtual nodes on `level` of a tree with leaf level L and vl virtual leaves:
// the leaf-level virtual suffix shrinks by halving (floor) per level upward.
TBVH_HD int virtual_at_level(int vl, int L, int level) { return vl >> (L - level); }

// Virtual nodes on all levels strictly above `level`:
//   sum_{j >= 1} (vl >> (L - level + j)) = 2x - popcount(x), x = vl >> (L-level+1).
TBVH_HD int virtual_above(int vl, int L, int level) {
    const uint32_t x = static_cast<uint32_t>(vl) >> (L - level + 1);
    return static_cast<int>(2u * x) - popcount(x);
}

TBVH_HD int real_at_level(int vl, int L, int level) {
    return (1 << level) - virtual_at_level(vl, L, level);
}

// Storage row of a real node given its heap index.
TBVH_HD int memory_index(int vl, int L, int i) {
    return i - virtual_above(vl, L, level_of(i));
}

TBVH_HD bool is_virtual(int vl, int L, int i) {
    const int level = level_of(i);
    return i - level_first(level) >= real_at_level(vl, L, level);
}

}  // namespace tree

// ---------------------------------------------------------------------------
// Morton codes (reference: morton.cuh:19-68).  Division is IEEE fp32 (this
// library is built without fast-math), so codes are a deterministic function
// of the inputs on every device.
// ---------------------------------------------------------------------------
namespace morton {

TBVH_HD float clamp_unit(float x) { return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x); }

// Position of x inside [lo, hi] as a fraction in [0, 1]; a degenerate or
// inverted extent maps everything to 0.
TBVH_HD float unit_coord(float x, float lo, float hi) {
    const float extent = hi - lo;
    if (extent <= 0.0f) return 0.0f;
    return clamp_unit((x - lo) / extent);
}

// Truncating quantisation into `bins` cells; the upper edge folds into the
// last cell.
TBVH_HD uint32_t cell(float u, uint32_t bins) {
    const float scaled = clamp_unit(u) * static_cast<float>(bins);
    const uint32_t c = static_cast<uint32_t>(scaled);
    return c >= bins ? bins - 1u : c;
}

// Spread the low 10 bits of v so bit b lands at bit 3b.
TBVH_HD uint32_t spread3(uint32_t v) {
    v &= 0x3ffu;
    v = (v | (v << 16)) & 0x030000ffu;
    v = (v | (v << 8)) & 0x0300f00fu;
    v = (v | (v << 4)) & 0x030c30c3u;
    v = (v | (v << 2)) & 0x09249249u;
    return v;
}

// Spread the low 16 bits of v so bit b lands at bit 2b.
TBVH_HD uint32_t spread2(uint32_t v) {
    v &= 0xffffu;
    v = (v | (v << 8)) & 0x00ff00ffu;
    v = (v | (v << 4)) & 0x0f0f0f0fu;
    v = (v | (v << 2)) & 0x33333333u;
    v = (v | (v << 1)) & 0x55555555u;
    return v;
}

// 30-bit (3-D, 1024 cells per axis) or 32-bit (2-D, 65536 cells per axis)
// code; axis 0 occupies the least significant interleaved bit.
template <int D>
TBVH_HD uint32_t encode(const float* p, const float* lo, const float* hi) {
    if constexpr (D == 3) {
        return spread3(cell(unit_coord(p[0], lo[0], hi[0]), 1024u)) |
               (spread3(cell(unit_coord(p[1], lo[1], hi[1]), 1024u)) << 1) |
               (spread3(cell(unit_coord(p[2], lo[2], hi[2]), 1024u)) << 2);
    } else {
        return spread2(cell(unit_coord(p[0], lo[0], hi[0]), 65536u)) |
               (spread2(cell(unit_coord(p[1], lo[1], hi[1]), 65536u)) << 1);
    }
}

template <int D>
constexpr int key_bits() { return D == 3 ? 30 : 32; }

}  // namespace morton

// ---------------------------------------------------------------------------
// Hilbert keys on the Morton grid (1024 cells per axis in 3-D, 65536 in 2-D),
// used only to order queries for traversal: consecutive keys are adjacent
// cells, so a wave's queries stay closer together than along the Z curve.
// Cell -> index follows J. Skilling, "Programming the Hilbert curve", AIP
// Conf. Proc. 707 (2004): the AxesToTranspose steps, then the transposed
// index read level by level from the top with axis 0 the most significant
// bit of each level.
//
// The traversal schedule sorts on the key's top 16 bits only.  Those are
// the index of the top 6 levels (3-D) or 8 levels (2-D): each step of the
// transform reads one bit level and rewrites only the levels below it, so
// the top levels of the index depend only on the top levels of the cell
// (the curve's self-similarity).  schedule_key therefore transforms just
// those levels of the cell and leaves the key's low bits zero: its top 16
// bits equal the full index's, at under half the work.
// ---------------------------------------------------------------------------
namespace hilbert {

// Index of the `b`-level cell x (b bits per axis; x is clobbered).
template <int D, int b>
TBVH_HD uint32_t index(uint32_t (&x)[D]) {
    // Inverse undo: reflect / exchange the lower levels, level by level.
#pragma unroll
    for (uint32_t q = 1u << (b - 1); q > 1u; q >>= 1) {
        const uint32_t m = q - 1u;
#pragma unroll
        for (int i = 0; i < D; ++i) {
            if (x[i] & q) {
                x[0] ^= m;
            } else {
                const uint32_t t = (x[0] ^ x[i]) & m;
                x[0] ^= t;
                x[i] ^= t;
            }
        }
    }
    // Gray encode.
#pragma unroll
    for (int i = 1; i < D; ++i) x[i] ^= x[i - 1];
    uint32_t t = 0u;
#pragma unroll
    for (uint32_t q = 1u << (b - 1); q > 1u; q >>= 1)
        if (x[D - 1] & q) t ^= q - 1u;
#pragma unroll
    for (int i = 0; i < D; ++i) x[i] ^= t;
    if constexpr (D == 3) {
        return morton::spread3(x[2]) | (morton::spread3(x[1]) << 1) | (morton::spread3(x[0]) << 2);
    } else {
        return morton::spread2(x[1]) | (morton::spread2(x[0]) << 1);
    }
}

// Schedule key: the top 16 bits of the Hilbert index of p's Morton cell in
// bits [key_bits - 16, key_bits), zeros below.
template <int D>
TBVH_HD uint32_t schedule_key(const float* p, const float* lo, const float* hi) {
    constexpr int b = D == 3 ? 10 : 16;      // levels of the full grid
    constexpr int top = D == 3 ? 6 : 8;      // levels that fix the top 16 bits
    uint32_t x[D];
#pragma unroll
    for (int d = 0; d < D; ++d) x[d] = morton::cell(morton::unit_coord(p[d], lo[d], hi[d]), 1u << b) >> (b - top);
    return index<D, top>(x) << (D * (b - top));
}

}  // namespace hilbert

// ---------------------------------------------------------------------------
// Segments.  Single, batched and ragged inputs are all a list of clouds
// ("segments") packed back to back; kernels index them through this table,
// which a planning kernel fills on the device from either (B, N) or device
// offsets.  Sort/partial tiles never straddle two segments.
// ---------------------------------------------------------------------------
constexpr int kSortTile = 4096;          // keys per sort/bounds tile
constexpr int kSubtreeLevels = 8;        // levels merged per tree-build pass
constexpr int kSubtreeLeaves = 1 << kSubtreeLevels;
constexpr int kMaxTreePasses = 4;        // ceil(31 / kSubtreeLevels)

struct Segment {
    int64_t start;        // first packed row (points or queries)
    int32_t n;            // rows in this segment
    int32_t tile_first;   // first sort tile of this segment
    int32_t tiles;        // sort tiles of this segment
    int32_t leaf_level;   // tree: L
    int32_t vl;           // tree: virtual leaves
    int32_t nr;           // tree: real nodes
    int64_t node_start;   // tree: first packed node row
    int32_t group_first[kMaxTreePasses];  // tree: first work-group per pass
    int32_t groups[kMaxTreePasses];       // tree: work-groups per pass
};

// Locate the segment whose [first, first + count) range holds `x`, given a
// monotone array of segment starts (`firsts[s]`, s < S).  Binary search for
// the last s with firsts[s] <= x.
template <typename T, typename F>
TBVH_HD int find_segment(F firsts, int S, T x) {
    int lo = 0, hi = S - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (firsts(mid) <= x) lo = mid; else hi = mid - 1;
    }
    return lo;
}

}  // namespace tbvh
