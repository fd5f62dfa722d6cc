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
// the listed nodes of kSpanGroups consecutive first-pass groups.  With one
// lane per node, each node's searches are a chain of dependent code loads
// (direction, exponential search, range search, split search: about
// 3 log2(extent)), up to 63 for the nodes near the root at 1M points, and
// the launch lasted as long as its longest chain (cfg2: 33 us for 34k
// nodes, 8 per first-pass group, most of them short).  So a lane takes a
// node only while its extent stays within kSpanLong positions (at most 8
// steps per search); longer nodes (18% at cfg2) are queued and taken by
// sub-groups of kSpanLanes lanes, where a search step probes 7 positions
// at once and resolves 3 bits, and the child boxes' cover rows load in one
// round trip.  Eight lanes for every node measured 18.5 us at cfg2 but
// slower at 4M points and more (a wave per node in every 8 turned a launch
// into several rounds of waves).
constexpr int kSpanLanes = 8;
constexpr int kSpanLong = 256;  // extents (positions from i) searched by one lane
// Calls of at most this many points give every node a sub-group
// (kSpanCoop): the waves still fit the chip in one round there, and the
// first phase's chains (up to 27 loads) no longer come before the queue's.
constexpr int64_t kSpanCoopPoints = int64_t(3) << 19;
template <bool kCoop>
constexpr int span_groups() { return kCoop ? 4 : 16; }

// The 8 bits of `v` over this lane's sub-group (lanes [base, base + 8) of
// the wave), lane base + j at bit j.
__device__ __forceinline__ uint32_t span_ballot(bool v) {
    const uint64_t m = __ballot(v);
    return static_cast<uint32_t>(m >> (lane_id() & ~(kSpanLanes - 1))) & ((1u << kSpanLanes) - 1);
}

// Largest m in [0, 2^p) with pred(m), for a predicate that holds at 0 and
// then fails from some point on: each step splits the interval into 8 (or
// fewer, for the last bits) parts and lane j tests the start of part j + 1.
template <class Pred>
__device__ __forceinline__ int span_search(int p, int sl, Pred pred) {
    int lo = 0;
    while (p > 0) {
        const int s3 = p < 3 ? p : 3;
        p -= s3;
        const int t = 1 << p;
        const bool probe = sl < (1 << s3) - 1;
        const uint32_t m = span_ballot(probe && pred(lo + (sl + 1) * t));
        lo += __popc(m) * t;
    }
    return lo;
}

// karras_node by one sub-group: the same direction, extent and split
// (every search below finds the boundary of a monotone predicate, which
// the one-lane binary searches find too), from global codes.  The
// exponential search starts at exponent p0 (prefix(i + 2^(p0 - 1) dir) >
// dmin is known).
__device__ __forceinline__ void span_karras_node(const CodeView& cv, int i, int sl, int p0, int& first, int& last,
                                                 int& gamma) {
    const uint32_t ci = cv.at(i);
    int dir, dmin;
    karras_dir(cv, i, ci, dir, dmin);
    // Exponential search: the first p >= p0 with prefix(i + 2^p dir) <=
    // dmin, 8 exponents per step (positions outside the cloud give -1).
    int p = p0;
    while (true) {
        const int e = p + sl;
        const uint32_t m = span_ballot(e < 30 && cv.prefix_len(i, ci, i + (1 << e) * dir) > dmin);
        if (m != (1u << kSpanLanes) - 1) {
            p += __builtin_ctz(~m);
            break;
        }
        p += kSpanLanes;
    }
    const int l = span_search(p, sl, [&](int m) { return cv.prefix_len(i, ci, i + m * dir) > dmin; });
    const int j = i + l * dir;
    const int dnode = cv.prefix_len(i, ci, j);
    const int split = span_search(p, sl, [&](int s) { return cv.prefix_len(i, ci, i + s * dir) > dnode; });
    gamma = i + split * dir + (dir < 0 ? dir : 0);
    first = min(i, j);
    last = max(i, j);
}

// range_box of [a0, b0] and [a1, b1] by one sub-group.  The cover visits
// at level u are those of range_box's loop in closed form: lo_u =
// ceil(lo / 2^u), hi_u = floor(hi / 2^u), row lo_u - 1 when lo_u is odd
// and row hi_u - 2 when hi_u is odd, while lo_u < hi_u.  Lane j loads the
// rows of levels j, j + 8, ... together, merges them, and the sub-group
// combines its lanes' boxes (min/max are exact and order-free on values).
template <int D>
__device__ __forceinline__ void span_range_boxes(const float* nodes, int vl, int L, int a0, int b0, int a1, int b1,
                                                 int sl, float* box0, float* box1) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
        box0[d] = FLT_MAX;
        box0[D + d] = -FLT_MAX;
        box1[d] = FLT_MAX;
        box1[D + d] = -FLT_MAX;
    }
    const int64_t top = int64_t(1) << L;
    const int64_t lo0 = a0 + top, hi0 = b0 + 1 + top, lo1 = a1 + top, hi1 = b1 + 1 + top;
    // Levels sl + 8k, k < 4, in two halves (all 32 levels at once held
    // 96 row floats in 3-D: 132 VGPRs); ranges below 2^16 points need only
    // the first half's round trip.
    constexpr int kRounds = 32 / kSpanLanes;
#pragma unroll
    for (int h = 0; h < kRounds; h += 2) {
        float r[2][4][2 * D];
        bool take[2][4];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int u = sl + (h + k) * kSpanLanes;
            const int64_t up = (int64_t(1) << u) - 1;
            const int64_t l0 = (lo0 + up) >> u, h0 = hi0 >> u, l1 = (lo1 + up) >> u, h1 = hi1 >> u;
            const int64_t row[4] = {l0 - 1, h0 - 2, l1 - 1, h1 - 2};
            take[k][0] = l0 < h0 && (l0 & 1);
            take[k][1] = l0 < h0 && (h0 & 1);
            take[k][2] = l1 < h1 && (l1 & 1);
            take[k][3] = l1 < h1 && (h1 & 1);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (take[k][c]) {
                    const float* src =
                        nodes + static_cast<int64_t>(tree::memory_index(vl, L, static_cast<int>(row[c]))) * 2 * D;
#pragma unroll
                    for (int f = 0; f < 2 * D; ++f) r[k][c][f] = src[f];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (take[k][0]) merge_row<D>(box0, r[k][0]);
            if (take[k][1]) merge_row<D>(box0, r[k][1]);
            if (take[k][2]) merge_row<D>(box1, r[k][2]);
            if (take[k][3]) merge_row<D>(box1, r[k][3]);
        }
    }
#pragma unroll
    for (int s = 1; s < kSpanLanes; s <<= 1) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            box0[d] = fminf(box0[d], __shfl_xor(box0[d], s, kWave));
            box0[D + d] = fmaxf(box0[D + d], __shfl_xor(box0[D + d], s, kWave));
            box1[d] = fminf(box1[d], __shfl_xor(box1[d], s, kWave));
            box1[D + d] = fmaxf(box1[D + d], __shfl_xor(box1[D + d], s, kWave));
        }
    }
}
template <int D, bool kCoop>
__global__ __launch_bounds__(kBlock) void accel_span_kernel(const Segment* __restrict__ segs, int S,
                                                            int64_t groups_bound,
                                                            const uint32_t* __restrict__ sorted_codes,
                                                            const uint32_t* __restrict__ span_list,
                                                            const uint32_t* __restrict__ span_count,
                                                            const float* __restrict__ node_aabbs,
                                                            float* __restrict__ records) {
    constexpr int R = 4 * D + 4;
    constexpr int kSpanGroups = span_groups<kCoop>();
    __shared__ int s_seg[kSpanGroups];
    __shared__ uint32_t s_base[kSpanGroups + 1];
    __shared__ int64_t s_list0[kSpanGroups];
    __shared__ uint32_t s_queue[kCoop ? 1 : kSpanGroups * kSubtreeLeaves];  // a group lists at most its own nodes
    __shared__ uint32_t s_queued;
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
    // Phase 1, one lane per node: direction and exponential search up to
    // kSpanLong positions; a node whose range reaches that far is queued for
    // phase 2, every other one finished here (searches of at most 8 steps).
    const auto node_of = [&](uint32_t e, Segment& g, int& i) {
        int k = 0;
        while (e >= s_base[k + 1]) ++k;
        g = segs[s_seg[k]];
        i = static_cast<int>(span_list[s_list0[k] + (e - s_base[k])]);
        return i >= 0 && i < g.n - 1;  // always, for entries the tree pass wrote
    };
    const auto view = [&](const Segment& g) {
        CodeView cv;
        cv.codes = sorted_codes + g.start;
        cv.win = nullptr;
        cv.w_lo = 0;
        cv.w_hi = 0;
        cv.n = g.n;
        return cv;
    };
    if (tid == 0) s_queued = kCoop ? s_base[kSpanGroups] : 0u;
    __syncthreads();
    for (uint32_t e = tid; !kCoop && e < s_base[kSpanGroups]; e += kBlock) {
        Segment g;
        int i;
        if (!node_of(e, g, i)) continue;
        const CodeView cv = view(g);
        const uint32_t ci = cv.at(i);
        int dir, dmin;
        karras_dir(cv, i, ci, dir, dmin);
        int lmax = 2;
        while (cv.prefix_len(i, ci, i + lmax * dir) > dmin) {
            lmax <<= 1;
            if (lmax > kSpanLong) break;
        }
        if (lmax > kSpanLong) {
            if constexpr (!kCoop) s_queue[atomicAdd(&s_queued, 1u)] = e;
            continue;
        }
        int first, last, gamma;
        karras_range(cv, i, ci, dir, dmin, lmax, first, last, gamma);
        // A node inside a bucket is never referenced; it must not write,
        // since its child links would overwrite the bucket's own link.
        if (i != 0 && last - first + 1 <= accel_bucket<D>()) continue;
        const float* nodes = node_aabbs + g.node_start * 2 * D;
        float lbox[2 * D], rbox[2 * D];
        range_box<D>(nodes, g.vl, g.leaf_level, first, gamma, lbox);
        range_box<D>(nodes, g.vl, g.leaf_level, gamma + 1, last, rbox);
        store_boxes<D>(records + (g.start + i) * R, lbox, rbox);
        link_record<D>(records + g.start * R, i, first, gamma, last);
    }
    __syncthreads();
    // Phase 2: sub-group `sub` (lanes sl = 0..7) takes queued nodes sub,
    // sub + 32, ... (kCoop: every listed node, from exponent 1); every
    // decision below is uniform over the sub-group.
    const int sub = tid / kSpanLanes;
    const int sl = tid % kSpanLanes;
    constexpr int kLongExp = __builtin_ctz(kSpanLong);
    for (uint32_t q = sub; q < s_queued; q += kBlock / kSpanLanes) {
        Segment g;
        int i;
        if (!node_of(kCoop ? q : s_queue[q], g, i)) continue;
        int first, last, gamma;
        span_karras_node(view(g), i, sl, kCoop ? 1 : kLongExp + 1, first, last, gamma);
        if (kCoop && i != 0 && last - first + 1 <= accel_bucket<D>()) continue;
        const float* nodes = node_aabbs + g.node_start * 2 * D;
        float lbox[2 * D], rbox[2 * D];
        span_range_boxes<D>(nodes, g.vl, g.leaf_level, first, gamma, gamma + 1, last, sl, lbox, rbox);
        if (sl == 0) {
            store_boxes<D>(records + (g.start + i) * R, lbox, rbox);
            link_record<D>(records + g.start * R, i, first, gamma, last);
        }
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
    auto run = [&](auto kernel, int groups) {
        kernel<<<static_cast<unsigned>((groups_bound + groups - 1) / groups), kBlock, 0, stream>>>(
            segs, Si, groups_bound, sorted_codes, span_list, span_count, node_aabbs, records);
    };
    const bool coop = total <= kSpanCoopPoints;
    if (D == 3) {
        coop ? run(accel_span_kernel<3, true>, span_groups<true>()) : run(accel_span_kernel<3, false>, span_groups<false>());
    } else {
        coop ? run(accel_span_kernel<2, true>, span_groups<true>()) : run(accel_span_kernel<2, false>, span_groups<false>());
    }
    return hipGetLastError();
}

}  // namespace tbvh
