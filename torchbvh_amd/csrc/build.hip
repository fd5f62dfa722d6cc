// BVH build kernels: segment planning, per-cloud bounds, Morton codes (with
// the first sort pass's tile histograms), implicit-tree node AABBs and the
// traversal arrays.
//
// Reference behaviour followed (torchbvh/csrc/bvh_build.cu):
//   bounds      :453-494  fminf/fmaxf from +-1e30 seeds, per cloud
//   Morton      :496-519  one u32 code per point against its cloud's bounds
//   node AABBs  :238-359  leaf = point box, parent = min/max of real children,
//                         single-real-child parent copies its child
//   traversal   :361-398  left/right child rows and leaf ranks per real node
// The work decomposition is this library's own: every kernel walks a table of
// segments (clouds), so single, batched and ragged inputs share one launch
// sequence, and the tree is built by level-synchronous LDS passes of
// 2^kSubtreeLevels nodes per work-group with no global atomics.
#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

template <typename T>
__device__ __forceinline__ T wave_inclusive_sum_t(T v) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const T o = __shfl_up(v, d, kWave);
        if (lane_id() >= d) v += o;
    }
    return v;
}

// 64-bit exclusive block prefix (one value per thread), with block total.
__device__ __forceinline__ int64_t block_exclusive_sum64(int64_t v, int64_t* scratch,
                                                         int64_t* total) {
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int64_t incl = wave_inclusive_sum_t<long long>(v);
    if (lane == kWave - 1) scratch[wave] = incl;
    __syncthreads();
    int64_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kBlock / kWave; ++w) {
        const int64_t t = scratch[w];
        before += (w < wave) ? t : 0;
        all += t;
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

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

__global__ __launch_bounds__(kBlock) void plan_uniform_kernel(Segment* segs, int64_t S, int n,
                                                              bool with_tree) {
    const int64_t s = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (s >= S) return;
    Segment g;
    fill_segment(g, s * n, n, with_tree);
    g.tile_first = static_cast<int32_t>(s * g.tiles);
    g.node_start = s * g.nr;
    for (int p = 0; p < kMaxTreePasses; ++p) g.group_first[p] = static_cast<int32_t>(s * g.groups[p]);
    segs[s] = g;
}

// One work-group scans all segments in chunks of kBlock.
__global__ __launch_bounds__(kBlock) void plan_offsets_kernel(Segment* segs, const int64_t* offsets,
                                                              int64_t S, bool with_tree,
                                                              int64_t* node_offsets) {
    __shared__ int64_t scratch[kBlock / kWave];
    int64_t carry_tiles = 0, carry_nodes = 0;
    int64_t carry_groups[kMaxTreePasses] = {0, 0, 0, 0};
    for (int64_t base = 0; base < S; base += kBlock) {
        const int64_t s = base + threadIdx.x;
        Segment g;
        const bool live = s < S;
        if (live) {
            const int64_t start = offsets[s];
            fill_segment(g, start, static_cast<int>(offsets[s + 1] - start), with_tree);
        } else {
            fill_segment(g, 0, 0, false);
            g.tiles = 0;
        }
        int64_t total;
        const int64_t tfirst = block_exclusive_sum64(live ? g.tiles : 0, scratch, &total);
        g.tile_first = static_cast<int32_t>(carry_tiles + tfirst);
        carry_tiles += total;
        const int64_t nfirst = block_exclusive_sum64(live ? g.nr : 0, scratch, &total);
        g.node_start = carry_nodes + nfirst;
        carry_nodes += total;
        for (int p = 0; p < kMaxTreePasses; ++p) {
            const int64_t gf = block_exclusive_sum64(live ? g.groups[p] : 0, scratch, &total);
            g.group_first[p] = static_cast<int32_t>(carry_groups[p] + gf);
            carry_groups[p] += total;
        }
        if (live) {
            segs[s] = g;
            if (node_offsets) node_offsets[s] = g.node_start;
        }
    }
    if (node_offsets && threadIdx.x == 0) node_offsets[S] = carry_nodes;
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
// Bounds
// ---------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(kBlock) void bounds_partial_kernel(const float* __restrict__ points,
                                                                const Segment* __restrict__ segs,
                                                                int S, float* __restrict__ partials) {
    __shared__ int s_seg;
    __shared__ float s_red[kBlock / kWave][2 * D];
    const int64_t t = blockIdx.x;
    const int s = block_find_segment([&](int i) { return static_cast<int64_t>(segs[i].tile_first); },
                                     S, t, &s_seg);
    const Segment g = segs[s];
    const int lt = static_cast<int>(t - g.tile_first);
    if (lt >= g.tiles) return;
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);

    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) { lo[d] = kSeedLo; hi[d] = kSeedHi; }
    for (int j = threadIdx.x; j < count; j += kBlock) {
        const float* p = points + (row0 + j) * D;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const float v = p[d];
            lo[d] = fminf(lo[d], v);
            hi[d] = fmaxf(hi[d], v);
        }
    }
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
        for (int w = 1; w < kBlock / kWave; ++w) v = c < D ? fminf(v, s_red[w][c]) : fmaxf(v, s_red[w][c]);
        partials[t * 2 * D + c] = v;
    }
}

template <int D>
__global__ __launch_bounds__(kBlock) void bounds_final_kernel(const Segment* __restrict__ segs,
                                                              const float* __restrict__ partials,
                                                              float* __restrict__ scene_min,
                                                              float* __restrict__ scene_max) {
    __shared__ float s_red[kBlock / kWave][2 * D];
    const int s = blockIdx.x;
    const Segment g = segs[s];
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) { lo[d] = kSeedLo; hi[d] = kSeedHi; }
    for (int j = threadIdx.x; j < g.tiles; j += kBlock) {
        const float* p = partials + (static_cast<int64_t>(g.tile_first) + j) * 2 * D;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            lo[d] = fminf(lo[d], p[d]);
            hi[d] = fmaxf(hi[d], p[D + d]);
        }
    }
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
        for (int w = 1; w < kBlock / kWave; ++w) v = c < D ? fminf(v, s_red[w][c]) : fmaxf(v, s_red[w][c]);
        if (c < D) scene_min[static_cast<int64_t>(s) * D + c] = v;
        else scene_max[static_cast<int64_t>(s) * D + c - D] = v;
    }
}

// ---------------------------------------------------------------------------
// Morton codes + digit-0 tile histograms
// ---------------------------------------------------------------------------
// Each wave walks its 1024-row slice of the tile in 16 rounds of 64 rows; the
// lanes that share a digit in a round are found with kRadixBits ballots and
// the lowest such lane bumps the wave's LDS counter for that digit.
template <int D>
__global__ __launch_bounds__(kBlock) void morton_kernel(const float* __restrict__ points,
                                                        const Segment* __restrict__ segs, int S,
                                                        const float* __restrict__ scene_min,
                                                        const float* __restrict__ scene_max,
                                                        uint32_t* __restrict__ keys,
                                                        uint32_t* __restrict__ hist,
                                                        uint32_t* __restrict__ dpre) {
    constexpr int kWaves = kBlock / kWave;
    constexpr int kItems = kSortTile / kBlock;
    __shared__ int s_seg;
    __shared__ uint32_t s_cnt[kWaves][kRadix];
    __shared__ uint32_t s_scan[kWaves];
    const int64_t t = blockIdx.x;
    const int s = block_find_segment([&](int i) { return static_cast<int64_t>(segs[i].tile_first); },
                                     S, t, &s_seg);
    const Segment g = segs[s];
    const int lt = static_cast<int>(t - g.tile_first);
    if (lt >= g.tiles) return;
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        lo[d] = scene_min[static_cast<int64_t>(s) * D + d];
        hi[d] = scene_max[static_cast<int64_t>(s) * D + d];
    }
    for (int i = threadIdx.x; i < kWaves * kRadix; i += kBlock) (&s_cnt[0][0])[i] = 0u;
    __syncthreads();

    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll 4
    for (int i = 0; i < kItems; ++i) {
        const int pos = wave * kWave * kItems + i * kWave + lane;
        const bool valid = pos < count;
        uint32_t code = 0xffffffffu;
        if (valid) {
            float p[D];
#pragma unroll
            for (int d = 0; d < D; ++d) p[d] = points[(row0 + pos) * D + d];
            code = morton::encode<D>(p, lo, hi);
            keys[row0 + pos] = code;
        }
        const uint32_t digit = code & (kRadix - 1);
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < kRadixBits; ++b) {
            const bool bit = (digit >> b) & 1u;
            const uint64_t m = __ballot(bit);
            peers &= bit ? m : ~m;
        }
        if (valid && (peers & below) == 0) s_cnt[wave][digit] += static_cast<uint32_t>(__popcll(peers));
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) c += s_cnt[w][threadIdx.x];
    const uint32_t excl = block_exclusive_sum(c, s_scan);
    const int64_t at = static_cast<int64_t>(kRadix) * g.tile_first +
                       static_cast<int64_t>(threadIdx.x) * g.tiles + lt;
    hist[at] = c;
    dpre[at] = excl;
}

// ---------------------------------------------------------------------------
// Implicit tree, level-synchronous passes
// ---------------------------------------------------------------------------
// Work-group `gl` of pass p owns 2^up consecutive nodes of level lvl_in
// (leaves for p == 0) and produces the `up` levels above them in LDS,
// writing every real node it forms.  Nodes of a level are contiguous in
// storage, so each level's writes are coalesced rows of 2D floats.
template <int D, bool kFromPoints>
__global__ __launch_bounds__(kBlock) void tree_pass_kernel(const float* __restrict__ points,
                                                           const Segment* __restrict__ segs, int S,
                                                           const int64_t* __restrict__ sorted,
                                                           float* __restrict__ node_aabbs, int p) {
    __shared__ int s_seg;
    __shared__ float s_box[(2 * kSubtreeLeaves - 1) * 2 * D];
    const int64_t grp = blockIdx.x;
    const int s = block_find_segment([&](int i) { return static_cast<int64_t>(segs[i].group_first[p]); },
                                     S, grp, &s_seg);
    const Segment g = segs[s];
    const int gl = static_cast<int>(grp - g.group_first[p]);
    if (gl >= g.groups[p]) return;
    const int L = g.leaf_level;
    const int vl = g.vl;
    const int lvl_in = L - p * kSubtreeLevels;
    const int up = lvl_in > kSubtreeLevels ? kSubtreeLevels : lvl_in;
    const int width = 1 << up;
    float* nodes = node_aabbs + g.node_start * 2 * D;
    const int tid = threadIdx.x;

    if (tid < width) {
        const int j = gl * width + tid;
        float* dst = s_box + (width - 1 + tid) * 2 * D;
        if (j < tree::real_at_level(vl, L, lvl_in)) {
            const int heap = tree::level_first(lvl_in) + j;
            const int64_t row = tree::memory_index(vl, L, heap);
            if constexpr (kFromPoints) {
                // Clamped so a corrupt permutation cannot read outside the cloud.
                const int64_t idx = min(max(sorted[g.start + j], int64_t(0)), int64_t(g.n - 1));
                const float* pt = points + (g.start + idx) * D;
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    const float v = pt[d];
                    dst[d] = v;
                    dst[D + d] = v;
                }
#pragma unroll
                for (int c = 0; c < 2 * D; ++c) nodes[row * 2 * D + c] = dst[c];
            } else {
#pragma unroll
                for (int c = 0; c < 2 * D; ++c) dst[c] = nodes[row * 2 * D + c];
            }
        }
    }
    __syncthreads();
    for (int step = 1; step <= up; ++step) {
        const int w = width >> step;
        if (tid < w) {
            const int lvl = lvl_in - step;
            const int j = gl * w + tid;
            if (j < tree::real_at_level(vl, L, lvl)) {
                const int heap = tree::level_first(lvl) + j;
                const int local = w - 1 + tid;
                const float* a = s_box + (2 * local + 1) * 2 * D;
                const float* b = a + 2 * D;
                const bool right_real = (2 * j + 1) < tree::real_at_level(vl, L, lvl + 1);
                float* dst = s_box + local * 2 * D;
#pragma unroll
                for (int d = 0; d < D; ++d) {
                    dst[d] = right_real ? fminf(a[d], b[d]) : a[d];
                    dst[D + d] = right_real ? fmaxf(a[D + d], b[D + d]) : a[D + d];
                }
                const int64_t row = tree::memory_index(vl, L, heap);
#pragma unroll
                for (int c = 0; c < 2 * D; ++c) nodes[row * 2 * D + c] = dst[c];
            }
        }
        __syncthreads();
    }
}

// One thread per stored node row: recover the heap index from the row and
// emit child rows (-1 for leaves / virtual right children) and leaf ranks.
__global__ __launch_bounds__(kBlock) void traversal_arrays_kernel(const Segment* __restrict__ segs,
                                                                  int S, int64_t total_nodes,
                                                                  int32_t* __restrict__ left,
                                                                  int32_t* __restrict__ right,
                                                                  int32_t* __restrict__ leaf) {
    const int64_t r = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (r >= total_nodes) return;
    const int s = find_segment([&](int i) { return segs[i].node_start; }, S, r);
    const Segment g = segs[s];
    const int lr = static_cast<int>(r - g.node_start);
    const int L = g.leaf_level;
    const int vl = g.vl;
    // Row range of level l starts at level_first(l) - virtual_above(l).
    int level = 0;
    while (level < L &&
           lr >= tree::level_first(level + 1) - tree::virtual_above(vl, L, level + 1)) {
        ++level;
    }
    const int heap = lr + tree::virtual_above(vl, L, level);
    if (level == L) {
        left[r] = -1;
        right[r] = -1;
        leaf[r] = heap - tree::level_first(L);
    } else {
        const int lc = 2 * heap + 1;
        const int rc = lc + 1;
        left[r] = tree::memory_index(vl, L, lc);
        right[r] = tree::is_virtual(vl, L, rc) ? -1 : tree::memory_index(vl, L, rc);
        leaf[r] = -1;
    }
}

inline unsigned grid_for(int64_t items) {
    return static_cast<unsigned>((items + kBlock - 1) / kBlock);
}

}  // namespace

hipError_t launch_plan_uniform(Segment* segs, int64_t S, int64_t n, bool tree, hipStream_t stream) {
    plan_uniform_kernel<<<grid_for(S), kBlock, 0, stream>>>(segs, S, static_cast<int>(n), tree);
    return hipGetLastError();
}

hipError_t launch_plan_offsets(Segment* segs, const int64_t* offsets, int64_t S, bool tree,
                               int64_t* node_offsets, hipStream_t stream) {
    plan_offsets_kernel<<<1, kBlock, 0, stream>>>(segs, offsets, S, tree, node_offsets);
    return hipGetLastError();
}

hipError_t launch_bounds(const float* points, int D, const Segment* segs, int64_t S,
                         int64_t tiles, float* partials, float* scene_min, float* scene_max,
                         hipStream_t stream) {
    if (D == 3) {
        bounds_partial_kernel<3><<<static_cast<unsigned>(tiles), kBlock, 0, stream>>>(
            points, segs, static_cast<int>(S), partials);
        bounds_final_kernel<3><<<static_cast<unsigned>(S), kBlock, 0, stream>>>(
            segs, partials, scene_min, scene_max);
    } else {
        bounds_partial_kernel<2><<<static_cast<unsigned>(tiles), kBlock, 0, stream>>>(
            points, segs, static_cast<int>(S), partials);
        bounds_final_kernel<2><<<static_cast<unsigned>(S), kBlock, 0, stream>>>(
            segs, partials, scene_min, scene_max);
    }
    return hipGetLastError();
}

hipError_t launch_morton(const float* points, int D, const Segment* segs, int64_t S, int64_t tiles,
                         const float* scene_min, const float* scene_max, uint32_t* keys,
                         uint32_t* hist, uint32_t* dpre, hipStream_t stream) {
    if (D == 3) {
        morton_kernel<3><<<static_cast<unsigned>(tiles), kBlock, 0, stream>>>(
            points, segs, static_cast<int>(S), scene_min, scene_max, keys, hist, dpre);
    } else {
        morton_kernel<2><<<static_cast<unsigned>(tiles), kBlock, 0, stream>>>(
            points, segs, static_cast<int>(S), scene_min, scene_max, keys, hist, dpre);
    }
    return hipGetLastError();
}

hipError_t launch_tree(const float* points, int D, const Segment* segs, int64_t S, int64_t total,
                       int64_t max_n, const int64_t* sorted, float* node_aabbs, hipStream_t stream) {
    // Passes needed by the deepest cloud.
    const int L = tree::leaf_level(static_cast<int>(max_n));
    const int passes = L == 0 ? 1 : (L + kSubtreeLevels - 1) / kSubtreeLevels;
    for (int p = 0; p < passes; ++p) {
        const int64_t groups = (total >> (kSubtreeLevels * (p + 1))) + S + 1;
        const unsigned grid = static_cast<unsigned>(groups);
        if (D == 3) {
            if (p == 0) tree_pass_kernel<3, true><<<grid, kBlock, 0, stream>>>(points, segs, static_cast<int>(S), sorted, node_aabbs, p);
            else tree_pass_kernel<3, false><<<grid, kBlock, 0, stream>>>(points, segs, static_cast<int>(S), sorted, node_aabbs, p);
        } else {
            if (p == 0) tree_pass_kernel<2, true><<<grid, kBlock, 0, stream>>>(points, segs, static_cast<int>(S), sorted, node_aabbs, p);
            else tree_pass_kernel<2, false><<<grid, kBlock, 0, stream>>>(points, segs, static_cast<int>(S), sorted, node_aabbs, p);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_traversal_arrays(const Segment* segs, int64_t S, int64_t total_nodes,
                                   int32_t* left, int32_t* right, int32_t* leaf,
                                   hipStream_t stream) {
    traversal_arrays_kernel<<<grid_for(total_nodes), kBlock, 0, stream>>>(
        segs, static_cast<int>(S), total_nodes, left, right, leaf);
    return hipGetLastError();
}

}  // namespace tbvh
