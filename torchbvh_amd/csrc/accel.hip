// k-NN acceleration structure derived from a finished implicit BVH.
//
// The implicit tree (the reference's payload, bit-exact) splits Morton-sorted
// points into fixed power-of-two runs; a run usually straddles a Morton cell
// boundary, so its box spans two cells and sibling boxes overlap heavily.  A
// radix tree over the same sorted codes (Karras, "Maximizing Parallelism in
// the Construction of BVHs, Octrees, and k-d Trees", HPG 2012) splits where
// the codes' common prefix ends, i.e. on Morton cell boundaries, and visits
// roughly ten times fewer nodes per query.  Because results are the k
// smallest (distance, index) pairs, the traversal structure cannot change
// them: this is a pure speed-up with identical output.
//
// Layout of one accel buffer (per cloud, clouds packed back to back):
//   points  [n]    float4 (x, y, z|0, original index as int bits), Morton order
//   records [n]    row i < n - 1: radix-tree internal node i: left box (2D
//                  floats), right box (2D floats), left ref, right ref,
//                  parent node (-1 at the root); every row's last word: the
//                  node whose record references the bucket that starts at
//                  point row i, if one does (row n - 1 holds only that word)
//                  (16 floats = 64 B in 3-D, 12 floats = 48 B in 2-D)
// A child ref >= 0 is an internal node; a negative ref is a bucket of at most
// accel_bucket<D>() (6 in 3-D, 8 in 2-D) consecutive points:
// 0x80000000 | (count - 1) << 28 | first.  Record rows follow point rows:
// cloud c's rows start at its first point row.  The parent links let the
// traversal resume exactly after its bounded stack dropped entries
// (knn.hip); words no node writes are never read.
//
// Child boxes are exact: each is the min/max over its point range, assembled
// from the implicit tree's node AABBs with an iterative segment-tree cover of
// the range (min/max is exact and idempotent), so no pass here needs
// cross-work-group synchronisation.
//
// Two ways to build it: the standalone passes below (points + codes, then
// one thread per node: tbvh_accel_build*), and the fused build
// (tbvh_build*_with_accel), where the first implicit-tree pass writes the
// points and the records of nodes inside each 256-leaf group and
// accel_span_kernel finishes the others.  Both produce the same bytes.
#include <float.h>

#include "accel_tree.hpp"

namespace tbvh {
namespace {

// Standalone pass 1: Morton-ordered points (float4) and their codes, one
// thread per point.
template <int D>
__global__ __launch_bounds__(kBlock) void accel_points_kernel(
    const float* __restrict__ points, const int64_t* __restrict__ sorted,
    const Segment* __restrict__ segs, int S, int64_t total, const float* __restrict__ scene_min,
    const float* __restrict__ scene_max, float4* __restrict__ leaf_points,
    uint32_t* __restrict__ codes) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (r >= total) return;
    const int s = find_segment([&](int i) { return segs[i].start; }, S, r);
    const Segment g = segs[s];
    const int64_t idx = min(max(sorted[r], int64_t(0)), int64_t(g.n - 1));
    float p[D], lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        p[d] = points[(g.start + idx) * D + d];
        lo[d] = scene_min[static_cast<int64_t>(s) * D + d];
        hi[d] = scene_max[static_cast<int64_t>(s) * D + d];
    }
    codes[r] = morton::encode<D>(p, lo, hi);
    float4 v;
    v.x = p[0];
    v.y = p[1];
    v.z = D == 3 ? p[D - 1] : 0.0f;
    v.w = __int_as_float(static_cast<int>(idx));
    leaf_points[r] = v;
}

// Standalone pass 1 from a finished implicit tree alone (no points, no
// bounds): leaf j of a cloud's tree is the degenerate box of its j-th point
// in Morton order, so the leaf rows give the Morton-ordered points, and the
// build's bounds follow exactly from the root box, which is the min / max
// over the same points: the build seeds its min at +1e30 and its max at
// -1e30 (bvh_build.cu:466-467), so scene_min = fminf(+1e30, root lo) and
// scene_max = fmaxf(-1e30, root hi).  The codes, and so the radix tree and
// every accel byte, are then the build's own.
template <int D>
__global__ __launch_bounds__(kBlock) void accel_points_from_tree_kernel(
    const float* __restrict__ node_aabbs, const int64_t* __restrict__ sorted, const Segment* __restrict__ segs,
    int S, int64_t total, float4* __restrict__ leaf_points, uint32_t* __restrict__ codes) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (r >= total) return;
    const int s = find_segment([&](int i) { return segs[i].start; }, S, r);
    const Segment g = segs[s];
    const int j = static_cast<int>(r - g.start);
    const float* nodes = node_aabbs + g.node_start * 2 * D;
    const int64_t row = tree::memory_index(g.vl, g.leaf_level, tree::level_first(g.leaf_level) + j);
    float p[D], lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        p[d] = nodes[row * 2 * D + d];
        lo[d] = fminf(kSeedLo, nodes[d]);
        hi[d] = fmaxf(kSeedHi, nodes[D + d]);
    }
    codes[r] = morton::encode<D>(p, lo, hi);
    const int64_t idx = min(max(sorted[r], int64_t(0)), int64_t(g.n - 1));
    float4 v;
    v.x = p[0];
    v.y = p[1];
    v.z = D == 3 ? p[D - 1] : 0.0f;
    v.w = __int_as_float(static_cast<int>(idx));
    leaf_points[r] = v;
}

// Whether a batched BVH known only by its node_aabbs and sorted_indices is a
// point BVH as the build writes it, which is what the pass above assumes:
// every leaf row a degenerate box (lo and hi bitwise equal, NaN included),
// every internal row the fminf/fmaxf merge of its children in the build's
// argument order (a copy of the left child where the right one is
// virtual), leaf codes non-decreasing against the root box's bounds, and
// sorted indices inside the cloud.  Then every accel child box is the exact
// box of its points and the accel answers exactly what the implicit tree
// answers.  One thread per node row (grid.y = cloud); any failure stores 1
// into *defects (every writer stores the same value), which the caller
// cleared first.
template <int D>
__global__ __launch_bounds__(kBlock) void tree_defects_kernel(const float* __restrict__ node_aabbs,
                                                              const int64_t* __restrict__ sorted, int n, int nr,
                                                              uint32_t* __restrict__ defects) {
    const int row = static_cast<int>(blockIdx.x) * kBlock + static_cast<int>(threadIdx.x);
    if (row >= nr) return;
    const int64_t b = blockIdx.y;
    const int L = tree::leaf_level(n);
    const int vl = tree::virtual_leaves(n);
    const float* nodes = node_aabbs + b * nr * 2 * D;
    // Rows hold the real nodes level by level; find this row's level.
    int level = 0;
    int level_row = 0;
    while (level < L && level_row + tree::real_at_level(vl, L, level) <= row) {
        level_row += tree::real_at_level(vl, L, level);
        ++level;
    }
    const float* box = nodes + static_cast<int64_t>(row) * 2 * D;
    bool bad = false;
    if (level == L) {
        const int j = row - level_row;
        float lo[D], hi[D], p[D], q[D];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            p[d] = box[d];
            bad |= __float_as_uint(box[d]) != __float_as_uint(box[D + d]);
            lo[d] = fminf(kSeedLo, nodes[d]);
            hi[d] = fmaxf(kSeedHi, nodes[D + d]);
        }
        const int64_t idx = sorted[b * n + j];
        bad |= idx < 0 || idx >= n;
        if (j > 0) {
#pragma unroll
            for (int d = 0; d < D; ++d) q[d] = box[d - 2 * D];
            bad |= morton::encode<D>(q, lo, hi) > morton::encode<D>(p, lo, hi);
        }
    } else {
        const int i = tree::level_first(level) + (row - level_row);
        const int left = 2 * i + 1;
        const bool right_real = !tree::is_virtual(vl, L, left + 1);
        const float* a = nodes + static_cast<int64_t>(tree::memory_index(vl, L, left)) * 2 * D;
        const float* c = a + 2 * D;  // the right sibling's row follows the left one's
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const float want_lo = right_real ? fminf(a[d], c[d]) : a[d];
            const float want_hi = right_real ? fmaxf(a[D + d], c[D + d]) : a[D + d];
            bad |= __float_as_uint(box[d]) != __float_as_uint(want_lo);
            bad |= __float_as_uint(box[D + d]) != __float_as_uint(want_hi);
        }
    }
    if (bad) *defects = 1u;
}

__global__ void clear_word_kernel(uint32_t* word) { *word = 0u; }

// Standalone pass 2: radix-tree internal nodes (Karras 2012, section 4), one
// thread per node; nodes inside a bucket are not referenced and write nothing.  The
// block first stages the sorted codes around its nodes in LDS (most nodes
// span few positions, so most of the searches' reads stay there; measured
// -5% in 3-D, -16% in 2-D).  Child boxes come from the implicit tree's node
// AABBs (reading the points directly measured slower, even for 16-point
// ranges: more bytes through L2).
constexpr int kCodeWindow = 2 * kBlock + 2 * kCodeHalo;
template <int D>
__global__ __launch_bounds__(kBlock) void accel_nodes_kernel(
    const Segment* __restrict__ segs, int S, int64_t total_points,
    const uint32_t* __restrict__ all_codes, const float* __restrict__ node_aabbs,
    float* __restrict__ records) {
    constexpr int R = 4 * D + 4;
    __shared__ uint32_t s_codes[kCodeWindow];
    __shared__ int64_t s_w0;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kBlock;
    const int64_t r = r0 + threadIdx.x;
    if (threadIdx.x == 0) {
        // Record row r is node r - start of the cloud holding point row r.
        const int64_t p0 = r0 - kCodeHalo;
        s_w0 = p0 < 0 ? 0 : p0;
    }
    __syncthreads();
    const int64_t w0 = s_w0;
    for (int k = threadIdx.x; k < kCodeWindow; k += kBlock) {
        const int64_t gp = w0 + k;
        s_codes[k] = gp < total_points ? all_codes[gp] : 0u;
    }
    __syncthreads();
    if (r >= total_points) return;
    const int s = find_segment([&](int c) { return segs[c].start; }, S, r);
    const Segment g = segs[s];
    const int n = g.n;
    const int i = static_cast<int>(r - g.start);
    if (i >= n - 1) return;
    // The window in positions of this cloud, clipped to it.
    CodeView cv;
    cv.codes = all_codes + g.start;
    cv.n = n;
    const int64_t lo = w0 - g.start;
    const int64_t hi = w0 + kCodeWindow - g.start;
    cv.win = s_codes + (lo > 0 ? 0 : -lo);
    cv.w_lo = static_cast<int>(lo > 0 ? lo : 0);
    cv.w_hi = static_cast<int>(hi < n ? (hi > 0 ? hi : 0) : n);
    int first, last, gamma;
    karras_node(cv, i, first, last, gamma);
    if (i != 0 && last - first + 1 <= accel_bucket<D>()) return;

    const float* nodes = node_aabbs + g.node_start * 2 * D;
    float* rec = records + r * R;
    float lbox[2 * D], rbox[2 * D];
    range_box<D>(nodes, g.vl, g.leaf_level, first, gamma, lbox);
    range_box<D>(nodes, g.vl, g.leaf_level, gamma + 1, last, rbox);
    store_boxes<D>(rec, lbox, rbox);
    link_record<D>(records + g.start * R, i, first, gamma, last);
}

// Records of the radix-tree nodes the fused first tree pass could not
// finish (their range spans two of its work-groups).  A work-group takes
// kSpanGroups consecutive first-pass groups and runs their listed nodes
// back to back, so its lanes stay busy; search and child boxes from global
// memory (the finished implicit tree).
constexpr int kSpanGroups = 8;
template <int D>
__global__ __launch_bounds__(kBlock) void accel_span_kernel(const Segment* __restrict__ segs, int S,
                                                            int64_t groups_bound,
                                                            const uint32_t* __restrict__ sorted_codes,
                                                            const uint32_t* __restrict__ span_list,
                                                            const uint32_t* __restrict__ span_count,
                                                            const float* __restrict__ node_aabbs,
                                                            float* __restrict__ records) {
    constexpr int R = 4 * D + 4;
    __shared__ int s_seg[kSpanGroups];
    __shared__ uint32_t s_base[kSpanGroups + 1];
    __shared__ int64_t s_list0[kSpanGroups];
    const int tid = threadIdx.x;
    if (tid < kSpanGroups) {
        const int64_t G = static_cast<int64_t>(blockIdx.x) * kSpanGroups + tid;
        uint32_t cnt = 0;
        int sg = 0;
        int64_t list0 = 0;
        if (G < groups_bound) {
            sg = find_segment([&](int c) { return static_cast<int64_t>(segs[c].group_first[0]); }, S, G);
            const Segment g = segs[sg];
            const int gl = static_cast<int>(G - g.group_first[0]);
            if (gl < g.groups[0]) {
                const int width = 1 << (g.leaf_level < kSubtreeLevels ? g.leaf_level : kSubtreeLevels);
                cnt = span_count[G];
                list0 = g.start + static_cast<int64_t>(gl) * width;
            }
        }
        s_seg[tid] = sg;
        s_list0[tid] = list0;
        s_base[tid + 1] = cnt;
    }
    __syncthreads();
    if (tid == 0) {
        s_base[0] = 0;
        for (int k = 1; k <= kSpanGroups; ++k) s_base[k] += s_base[k - 1];
    }
    __syncthreads();
    for (uint32_t e = tid; e < s_base[kSpanGroups]; e += kBlock) {
        int k = 0;
        while (e >= s_base[k + 1]) ++k;
        const int sg = s_seg[k];
        const Segment g = segs[sg];
        const int i = static_cast<int>(span_list[s_list0[k] + (e - s_base[k])]);
        if (i < 0 || i >= g.n - 1) continue;  // never for entries the tree pass wrote
        CodeView cv;
        cv.codes = sorted_codes + g.start;
        cv.win = nullptr;
        cv.w_lo = 0;
        cv.w_hi = 0;
        cv.n = g.n;
        int first, last, gamma;
        karras_node(cv, i, first, last, gamma);
        // A node inside a bucket is never referenced; it must not write,
        // since its child links would overwrite the bucket's own link.
        if (i != 0 && last - first + 1 <= accel_bucket<D>()) continue;
        const float* nodes = node_aabbs + g.node_start * 2 * D;
        float* rec = records + (g.start + i) * R;
        float lbox[2 * D], rbox[2 * D];
        range_box<D>(nodes, g.vl, g.leaf_level, first, gamma, lbox);
        range_box<D>(nodes, g.vl, g.leaf_level, gamma + 1, last, rbox);
        store_boxes<D>(rec, lbox, rbox);
        link_record<D>(records + g.start * R, i, first, gamma, last);
    }
}

inline unsigned grid_for(int64_t items) {
    return static_cast<unsigned>((items + kBlock - 1) / kBlock);
}

}  // namespace

size_t accel_bytes(int64_t total, int64_t /*S*/, int D) {
    return accel_points_bytes(total) + static_cast<size_t>(total) * (4 * D + 4) * sizeof(float);
}

hipError_t launch_accel_points(const float* points, const int64_t* sorted, const float* scene_min,
                               const float* scene_max, int D, const Segment* segs, int64_t S,
                               int64_t total, uint32_t* codes, void* accel, hipStream_t stream) {
    float4* leaf_points = static_cast<float4*>(accel);
    const int Si = static_cast<int>(S);
    if (D == 3) {
        accel_points_kernel<3><<<grid_for(total), kBlock, 0, stream>>>(
            points, sorted, segs, Si, total, scene_min, scene_max, leaf_points, codes);
    } else {
        accel_points_kernel<2><<<grid_for(total), kBlock, 0, stream>>>(
            points, sorted, segs, Si, total, scene_min, scene_max, leaf_points, codes);
    }
    return hipGetLastError();
}

hipError_t launch_accel_points_from_tree(const float* node_aabbs, const int64_t* sorted, int D,
                                         const Segment* segs, int64_t S, int64_t total, uint32_t* codes,
                                         void* accel, hipStream_t stream) {
    float4* leaf_points = static_cast<float4*>(accel);
    const int Si = static_cast<int>(S);
    if (D == 3) {
        accel_points_from_tree_kernel<3><<<grid_for(total), kBlock, 0, stream>>>(node_aabbs, sorted, segs, Si, total,
                                                                                 leaf_points, codes);
    } else {
        accel_points_from_tree_kernel<2><<<grid_for(total), kBlock, 0, stream>>>(node_aabbs, sorted, segs, Si, total,
                                                                                 leaf_points, codes);
    }
    return hipGetLastError();
}

hipError_t launch_tree_defects(const float* node_aabbs, const int64_t* sorted, int D, int64_t B, int n, int nr,
                               uint32_t* defects, hipStream_t stream) {
    clear_word_kernel<<<1, 1, 0, stream>>>(defects);
    const dim3 grid(grid_for(nr), static_cast<unsigned>(B));
    if (D == 3) {
        tree_defects_kernel<3><<<grid, kBlock, 0, stream>>>(node_aabbs, sorted, n, nr, defects);
    } else {
        tree_defects_kernel<2><<<grid, kBlock, 0, stream>>>(node_aabbs, sorted, n, nr, defects);
    }
    return hipGetLastError();
}

hipError_t launch_accel_nodes(const float* node_aabbs, int D, const Segment* segs, int64_t S,
                              int64_t total, const uint32_t* sorted_codes, void* accel,
                              hipStream_t stream) {
    if (total - S <= 0) return hipSuccess;
    float* records = reinterpret_cast<float*>(static_cast<char*>(accel) + accel_points_bytes(total));
    const int Si = static_cast<int>(S);
    if (D == 3) {
        accel_nodes_kernel<3><<<grid_for(total), kBlock, 0, stream>>>(segs, Si, total, sorted_codes, node_aabbs,
                                                                      records);
    } else {
        accel_nodes_kernel<2><<<grid_for(total), kBlock, 0, stream>>>(segs, Si, total, sorted_codes, node_aabbs,
                                                                      records);
    }
    return hipGetLastError();
}

hipError_t launch_accel_span(const float* node_aabbs, int D, const Segment* segs, int64_t S, int64_t total,
                             int64_t groups_bound, const uint32_t* sorted_codes, const uint32_t* span_list,
                             const uint32_t* span_count, void* accel, hipStream_t stream) {
    if (total - S <= 0) return hipSuccess;
    float* records = reinterpret_cast<float*>(static_cast<char*>(accel) + accel_points_bytes(total));
    const int Si = static_cast<int>(S);
    const unsigned grid = static_cast<unsigned>((groups_bound + kSpanGroups - 1) / kSpanGroups);
    if (D == 3) {
        accel_span_kernel<3><<<grid, kBlock, 0, stream>>>(segs, Si, groups_bound, sorted_codes, span_list,
                                                          span_count, node_aabbs, records);
    } else {
        accel_span_kernel<2><<<grid, kBlock, 0, stream>>>(segs, Si, groups_bound, sorted_codes, span_list,
                                                          span_count, node_aabbs, records);
    }
    return hipGetLastError();
}

}  // namespace tbvh
