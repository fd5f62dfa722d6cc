// Internal (non-ABI) declarations shared by the HIP translation units:
// wavefront helpers and the host-side launchers each unit provides.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "tbvh_common.hpp"

namespace tbvh {

constexpr int kWave = 64;     // CDNA wavefront width
constexpr int kBlock = 256;   // default threads per work-group (kernels with other shapes say so)
constexpr int kRadixBits = 8;
constexpr int kRadix = 1 << kRadixBits;
constexpr float kSeedLo = 1.0e30f;   // bounds seeds (reference: bvh_build.cu:466-467)
constexpr float kSeedHi = -1.0e30f;

// ---------------------------------------------------------------------------
// Wavefront / work-group helpers (device)
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return static_cast<int>(__lane_id()); }

__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t v) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t o = __shfl_up(v, d, kWave);
        if (lane_id() >= d) v += o;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v = fminf(v, __shfl_xor(v, d, kWave));
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, kWave));
    return v;
}

// Exclusive prefix sum of one value per thread over a kThreads-thread group.
// `scratch` must hold kThreads / kWave words.  Contains __syncthreads().
template <int kThreads = kBlock>
__device__ __forceinline__ uint32_t block_exclusive_sum(uint32_t v, uint32_t* scratch,
                                                        uint32_t* total = nullptr) {
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const uint32_t incl = wave_inclusive_sum(v);
    if (lane == kWave - 1) scratch[wave] = incl;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) {
        const uint32_t t = scratch[w];
        before += (w < wave) ? t : 0u;
        all += t;
    }
    __syncthreads();
    if (total) *total = all;
    return before + incl - v;
}

// Segment owning work item `x` of a per-segment range table, found by one
// thread and broadcast through LDS.
template <typename F>
__device__ __forceinline__ int block_find_segment(F firsts, int S, int64_t x, int* s_seg) {
    if (threadIdx.x == 0) *s_seg = find_segment(firsts, S, x);
    __syncthreads();
    return *s_seg;
}

// ---------------------------------------------------------------------------
// Segment tables (device): each cloud's rows, tiles, tree sizes and the
// work-groups of each tree pass, filled in closed form for equal clouds.
// ---------------------------------------------------------------------------
// How the first launch of a sequence finds its segments: for S equal
// clouds of n rows (n > 0) it computes each one in place, and also stores
// the whole table into `table` for the launches after it (so no planning
// launch runs first); with n == 0 it reads the table a planning launch
// filled.
struct UniformPlan {
    Segment* table = nullptr;
    int n = 0;
    bool tree = false;
};

// Work-groups of tree pass p for one cloud: pass p merges up to
// kSubtreeLevels levels starting at level L - p*kSubtreeLevels; one group per
// real node of the level it stops at.  Inactive passes have zero groups.
__host__ __device__ inline int tree_pass_groups(int L, int vl, int p) {
    const int lvl_in = L - p * kSubtreeLevels;
    if (p > 0 && lvl_in <= 0) return 0;
    const int top = lvl_in > kSubtreeLevels ? lvl_in - kSubtreeLevels : 0;
    return tree::real_at_level(vl, L, top);
}

__device__ inline void fill_segment(Segment& g, int64_t start, int n, bool with_tree) {
    g.start = start;
    g.n = n;
    g.tiles = (n + kSortTile - 1) / kSortTile;
    if (with_tree) {
        g.leaf_level = tree::leaf_level(n);
        g.vl = tree::virtual_leaves(n);
        g.nr = tree::real_node_count(n);
        for (int p = 0; p < kMaxTreePasses; ++p) g.groups[p] = tree_pass_groups(g.leaf_level, g.vl, p);
    } else {
        g.leaf_level = 0;
        g.vl = 0;
        g.nr = 0;
        for (int p = 0; p < kMaxTreePasses; ++p) g.groups[p] = 0;
    }
}

// Segment i of S equal clouds of n rows.
__device__ inline Segment uniform_segment(int64_t i, int n, bool with_tree) {
    Segment g;
    fill_segment(g, i * n, n, with_tree);
    g.tile_first = static_cast<int32_t>(i * g.tiles);
    g.node_start = i * g.nr;
    for (int p = 0; p < kMaxTreePasses; ++p) g.group_first[p] = static_cast<int32_t>(i * g.groups[p]);
    return g;
}

// Grid-stride store of the whole table of S equal clouds.
__device__ inline void store_uniform_table(Segment* segs, int64_t S, int n, bool with_tree) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < S; i += stride) {
        segs[i] = uniform_segment(i, n, with_tree);
    }
}

// Segment of tile t in the first launch of a sequence (see UniformPlan):
// computed for equal clouds (tiles past the last cloud's count as surplus
// tiles of it), else looked up in the table.  Ends with a barrier either way.
__device__ inline Segment first_launch_segment(const Segment* segs, int S, const UniformPlan& plan, int64_t t,
                                               int* s_seg, int* seg_out) {
    if (plan.n > 0) {
        const int64_t per = (plan.n + kSortTile - 1) / kSortTile;
        const int s = static_cast<int>(min(t / per, static_cast<int64_t>(S) - 1));
        __syncthreads();
        *seg_out = s;
        return uniform_segment(s, plan.n, plan.tree);
    }
    const int s = block_find_segment([&](int i) { return static_cast<int64_t>(segs[i].tile_first); }, S, t, s_seg);
    *seg_out = s;
    return segs[s];
}

// Block-wide min (c < D) / max (c >= D) of per-thread boxes; the result for
// component c lands in out[c] for threads c < 2D.
template <int D, int kThreads = kBlock>
__device__ __forceinline__ void block_box(float (&lo)[D], float (&hi)[D], float (*s_red)[2 * D],
                                          float* out) {
    const int wave = threadIdx.x / kWave;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        lo[d] = wave_min(lo[d]);
        hi[d] = wave_max(hi[d]);
    }
    if (lane_id() == 0) {
#pragma unroll
        for (int d = 0; d < D; ++d) { s_red[wave][d] = lo[d]; s_red[wave][D + d] = hi[d]; }
    }
    __syncthreads();
    if (threadIdx.x < 2 * D) {
        const int c = threadIdx.x;
        float v = s_red[0][c];
        for (int w = 1; w < kThreads / kWave; ++w) v = c < D ? fminf(v, s_red[w][c]) : fmaxf(v, s_red[w][c]);
        out[c] = v;
    }
}

// Whole points as one load per lane (dwordx3 / dwordx2: a wave reads 64
// consecutive points).
template <int D>
struct PointRow {
    float v[D];
};

// Lanes of the current wave holding the same digit as this lane (among
// `valid` lanes).
__device__ __forceinline__ uint64_t match_digit(uint32_t digit, bool valid) {
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < kRadixBits; ++b) {
        const bool bit = (digit >> b) & 1u;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

// ---------------------------------------------------------------------------
// Launchers (host).  Every launcher enqueues on `stream` and returns the
// launch status.
// ---------------------------------------------------------------------------

// Sort scratch: ping-pong keys/values; the current pass's digit count of
// every tile and its exclusive scan along the tiles, both digit-major
// ([digit][tile], row stride `tstride`).  Nothing needs clearing.
struct SortBuffers {
    uint32_t* keys_a;     // input keys (Morton kernel output)
    uint32_t* keys_b;
    uint32_t* vals_a;
    uint32_t* vals_b;
    uint32_t* tile_hist;  // kRadix * tstride words
    uint32_t* tile_scan;  // kRadix * tstride words
    int64_t tstride;      // >= tiles_bound, a multiple of 64
};

// Row stride of the digit-major tile arrays.
inline int64_t tile_stride(int64_t tiles_bound) { return (tiles_bound + 63) / 64 * 64; }

// One scatter pass (device-side view).
struct SortPass {
    const uint32_t* keys_in;
    const uint32_t* vals_in;
    uint32_t* keys_out;
    uint32_t* vals_out;
    int64_t* idx_out;
    const uint32_t* tile_scan;  // [digit][tile], exclusive along tiles
    int64_t tstride;
    int shift;
};


// Planning: fill the segment table.
hipError_t launch_plan_uniform(Segment* segs, int64_t S, int64_t n, bool tree, hipStream_t stream);
hipError_t launch_plan_offsets(Segment* segs, const int64_t* offsets, int64_t S, bool tree,
                               int64_t* node_offsets, hipStream_t stream);

// Per-cloud bounds: one work-group per tile writes a partial box
// (`partials`: 2D floats per tile); with `finalize`, one work-group per
// cloud then reduces them into scene_min/max (otherwise launch_morton does,
// given the same partials in a BoundsFinish).
hipError_t launch_bounds(const float* points, int D, const Segment* segs, int64_t S,
                         int64_t tiles_bound, float* partials, float* scene_min, float* scene_max,
                         bool finalize, float seed_lo, float seed_hi, UniformPlan plan, hipStream_t stream);

// Clouds of at most this many tiles get their bounds reduced inside the
// Morton kernel (each of a cloud's work-groups reads all its partial boxes,
// so the reads grow with the square of its tile count); larger ones take
// the separate per-cloud reduction.
constexpr int64_t kFuseBoundsTiles = 1024;

// Bounds still to reduce when keys are computed: the partial boxes and the
// seeds of the reduction (partials null: scene_min/max are final already).
struct BoundsFinish {
    const float* partials = nullptr;
    float seed_lo = 0.0f;
    float seed_hi = 0.0f;
};

// Digit range of a sort: 8-bit digits at bits first_bit, first_bit + 8, ...
// below end_bit (so passes = ceil((end_bit - first_bit) / 8) <= 4), and the
// curve launch_morton keys rows on (Hilbert only for the query schedule).
struct SortBits {
    int first_bit;
    int end_bit;
    bool hilbert = false;
    int passes() const { return (end_bit - first_bit + kRadixBits - 1) / kRadixBits; }
};

// Clouds of at most kSmallCloud rows (small.hip): one work-group per cloud
// computes its bounds (with `bounds`, from the seeds; else reads
// scene_min/max), its keys (the curve of `bits`) and the whole stable sort in
// LDS, and writes the cloud-local order and, if given, the sorted keys:
// what launch_bounds + launch_morton + launch_sort produce, in one launch.
// `max_n` bounds every cloud's row count (>= 1).
constexpr int64_t kSmallCloud = 12288;
hipError_t launch_small_sort(const float* rows, int D, const Segment* segs, int64_t S, UniformPlan plan,
                             int64_t max_n, float* scene_min, float* scene_max, bool bounds, float seed_lo,
                             float seed_hi, SortBits bits, int64_t* order, uint32_t* sorted_keys,
                             hipStream_t stream);

// Primitive BVH input: every primitive's box and centre, and each cloud's
// bounds over the boxes (partials as in launch_bounds).
hipError_t launch_primitive_prep(const float* prims, int D, int V, const Segment* segs, int64_t S,
                                 int64_t tiles, float* centers, float* boxes, float* partials,
                                 float* scene_min, float* scene_max, bool finalize, hipStream_t stream);

// Morton (or, with bits.hilbert, Hilbert) keys of every row against its
// segment's bounds and, unless `tile_hist` is null, every tile's count of
// the first sort digit (digit at bits.first_bit; [digit][tile], row stride
// `tstride`, surplus tiles zero).  With fin.partials the bounds are first
// reduced from the partial boxes and stored into scene_min/max.
hipError_t launch_morton(const float* points, int D, const Segment* segs, int64_t S,
                         int64_t tiles_bound, float* scene_min, float* scene_max,
                         uint32_t* keys, uint32_t* tile_hist, int64_t tstride, SortBits bits,
                         BoundsFinish fin, hipStream_t stream, UniformPlan plan = UniformPlan{});

// Stable LSD sort of (key, local index) per segment on the digits of
// `bits`; writes int64 local indices in key order into `order` and, if
// `sorted_keys` is non-null, the keys in that order (an even number of
// passes leaves them in buf.keys_a).  Input keys are in buf.keys_a
// (clobbered); buf.tile_hist holds the first digit's tile counts (written
// by the key producer, launch_morton or launch_route_keys).
hipError_t launch_sort(const Segment* segs, int64_t S, int64_t tiles_bound, SortBits bits,
                       const SortBuffers& buf, int64_t* order, uint32_t* sorted_keys,
                       hipStream_t stream);

// Extra outputs of the implicit-tree passes.
struct TreeOutputs {
    int32_t* left;         // traversal arrays (null: not written)
    int32_t* right;
    int32_t* leaf;
    bool arrays_packed;    // ragged: per-segment arrays at node_start; batched: segment 0 only
    float4* accel_points;  // Morton-ordered float4 points for the accel (null: not written)
    const float* leaf_boxes = nullptr;  // primitive BVH: [rows, 2D] leaf boxes (null: point leaves)
    // Fused accel records (first pass): with `sorted_codes` set, every
    // radix-tree node of a work-group's leaves whose range lies inside the
    // group gets its record in `accel_records`; the others are listed for
    // launch_accel_span: node indices compacted in the group's own record
    // rows of `span_list`, their count per first-pass work-group in
    // `span_count`.
    const uint32_t* sorted_codes = nullptr;
    float* accel_records = nullptr;
    uint32_t* span_list = nullptr;   // one word per record row
    uint32_t* span_count = nullptr;  // one word per first-pass work-group
};

// Implicit-tree node AABBs (all passes), optionally the traversal arrays and
// the accel's points.  `max_n` bounds the largest cloud (it decides how
// many passes run).
hipError_t launch_tree(const float* points, int D, const Segment* segs, int64_t S,
                       int64_t total, int64_t max_n, const int64_t* sorted, float* node_aabbs,
                       const TreeOutputs& out, hipStream_t stream);

// k-NN acceleration structure (radix tree + Morton-ordered float4 points).
// Max points per leaf bucket (bucket refs hold count - 1 in 3 bits).
// Measured on MI355X with the min/max candidate insertion: 3-D 6 against 4:
// -11% at cfg3, -1% at cfg2 and cfg5 (5 and 7: slower than 6 at cfg2, 8:
// +22% at cfg5); 2-D 8 is 8% faster than 4 (cfg4), 6 slower than 8.
template <int D>
__host__ __device__ constexpr int accel_bucket() { return D == 2 ? 8 : 6; }
constexpr int64_t kMaxAccelCloud = int64_t(1) << 28;  // bucket refs hold 28-bit starts
__host__ __device__ inline size_t accel_points_bytes(int64_t total) {
    return (static_cast<size_t>(total) * 16 + 255) / 256 * 256;
}
size_t accel_bytes(int64_t total, int64_t S, int D);
// Accel points + codes from a finished BVH (`codes`: scratch for `total`
// u32), then the radix-tree records.
hipError_t launch_accel_points(const float* points, const int64_t* sorted, const float* scene_min,
                               const float* scene_max, int D, const Segment* segs, int64_t S,
                               int64_t total, uint32_t* codes, void* accel, hipStream_t stream);
// Accel points + codes from a finished implicit tree alone (its leaf rows
// and root box), identical to launch_accel_points' for the same build.
hipError_t launch_accel_points_from_tree(const float* node_aabbs, const int64_t* sorted, int D,
                                         const Segment* segs, int64_t S, int64_t total, uint32_t* codes,
                                         void* accel, hipStream_t stream);
// Clears *defects, then sets it to 1 unless the B clouds' node_aabbs
// ([B, nr, 2D]) and sorted_indices ([B, n]) form the point BVH the build
// writes (what launch_accel_points_from_tree assumes).
hipError_t launch_tree_defects(const float* node_aabbs, const int64_t* sorted, int D, int64_t B, int n, int nr,
                               uint32_t* defects, hipStream_t stream);
// Records of the nodes the fused first tree pass listed (after all tree
// passes: their boxes need the upper levels).  `groups_bound` bounds the
// first pass's work-group count.
hipError_t launch_accel_span(const float* node_aabbs, int D, const Segment* segs, int64_t S, int64_t total,
                             int64_t groups_bound, const uint32_t* sorted_codes, const uint32_t* span_list,
                             const uint32_t* span_count, void* accel, hipStream_t stream);
// Radix-tree records from Morton-sorted codes and the implicit tree.
hipError_t launch_accel_nodes(const float* node_aabbs, int D, const Segment* segs, int64_t S,
                              int64_t total, const uint32_t* sorted_codes, void* accel,
                              hipStream_t stream);

// Routed query ordering (route.hip): route digits + their tile counts;
// partitioned queries, 2B group segments and bounds (a cloud's false count
// from the route sort's tile scan); final query order.
hipError_t launch_route_keys(const uint8_t* routes, const Segment* segs, int64_t S, int64_t tiles,
                             uint32_t* keys, uint32_t* tile_hist, int64_t tstride, hipStream_t stream);
hipError_t launch_route_gather(const float* queries, const int64_t* part, const Segment* segs,
                               const uint32_t* tile_scan, int64_t B,
                               int64_t M, int D, const float* true_min, const float* true_max,
                               const float* false_min, const float* false_max, float* gathered,
                               int64_t* group_offsets, float* group_min, float* group_max,
                               hipStream_t stream);
hipError_t launch_route_finish(const int64_t* part, const int64_t* sorted_local, const int64_t* group_offsets,
                               int64_t B, int64_t M, int64_t* order, hipStream_t stream);

// interpolate_displaced's rank loop and exact-hit select, one thread per
// (query row, channel group); writes the (rows, C) result.
hipError_t launch_interpolate(const float* values, const int64_t* indices, const float* weights,
                              const uint8_t* exact, int64_t rows, int64_t N, int64_t H, int64_t C, int K,
                              float* out, hipStream_t stream);

// k-NN traversal.
struct KnnArgs {
    const float* node_aabbs;
    const int64_t* sorted_indices;
    const float* queries;
    const int64_t* order;          // may be null
    const int64_t* point_offsets;  // ragged only
    const int64_t* node_offsets;   // ragged only
    const int64_t* query_offsets;  // ragged only
    int64_t B;
    int64_t M;                     // batched: queries per cloud
    int64_t total_q;
    int32_t num_leaves;            // batched only
    int32_t num_real_nodes;        // batched only
    int64_t* out_indices;
    float* out_distances;
    const void* accel;             // accelerated traversal only
    int64_t total_points;          // accelerated traversal only
    bool spatial_output;           // write row `launch position` instead of `query index`
    // Fused neighbour rows: with out_positions set, row j of a result also
    // gets the source_points row of neighbour j (source_cols floats; the
    // source has the points' layout, so a cloud's rows start where its
    // points do).  Not with routes.
    const float* source_points;
    int32_t source_cols;
    float* out_positions;
    // Routed traversal (batched only): a query whose route is false searches
    // the second structure and its indices are offset by num_leaves.
    const uint8_t* routes;         // null: not routed
    const float* node_aabbs2;      // implicit tree of the false route
    const int64_t* sorted_indices2;
    const void* accel2;            // accel of the false route
    int32_t num_leaves2;
    int32_t num_real_nodes2;
    // Fallback pass of the cell-block search (batched accel only): the list
    // is sub-lists of fb_seg entries, each with a count in fb_count (knn.hip
    // grid_sublist); an entry names a launch position, whose query runs with
    // its list seeded with the k-th distance bound fb_bound[position]
    // (FLT_MAX: none).
    const int32_t* fb_list;
    const float* fb_bound;
    const uint32_t* fb_count;
    int64_t fb_seg;
};
hipError_t launch_knn(const KnnArgs& a, int D, int K, bool ragged, hipStream_t stream);
hipError_t launch_knn_accel(const KnnArgs& a, int D, int K, bool ragged, hipStream_t stream);

// Cell-block k-NN (batched accel, `a` as for launch_knn_accel; spatial
// output and neighbour rows as there): every cloud's accel points are cut
// into the level-`level` Morton cells against its root box (row 0 of its
// node_aabbs, `nr` rows per cloud); each query scans the 3^D cells around
// its own and keeps the result when its k-th distance is inside the
// block's margin; the others run the accel traversal seeded with that
// distance.  Routed (a.routes set: ordered, spatial output, no neighbour
// rows): the false route's structure has its own boxes (node_aabbs2, nr2
// rows per cloud) and level (level2 >= 2), and each query searches its
// route's; level2 = 0 otherwise.  `ws` holds grid_workspace_bytes(B,
// total_q, level, D, level2).
int grid_level(int64_t n, int D, int K);
size_t grid_workspace_bytes(int64_t B, int64_t total_q, int level, int D, int level2 = 0);
hipError_t launch_grid_knn(const KnnArgs& a, const float* node_aabbs, int64_t nr, int level, int D, int K,
                           void* ws, hipStream_t stream, const float* node_aabbs2 = nullptr, int64_t nr2 = 0,
                           int level2 = 0);

// Tile-count bound for S segments holding `total` rows in kSortTile tiles.
inline int64_t tiles_bound(int64_t total, int64_t S) {
    return (total + kSortTile - 1) / kSortTile + S;
}

}  // namespace tbvh
