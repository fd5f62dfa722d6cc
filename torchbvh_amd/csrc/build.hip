// BVH build kernels: segment planning, per-cloud bounds, Morton codes (with
// the first sort digit's tile counts), implicit-tree node AABBs, fused with
// the traversal arrays and, when requested, the k-NN accel's Morton-ordered
// points and the radix-tree records of nodes inside each 256-leaf group.
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
#include "accel_tree.hpp"

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

__global__ __launch_bounds__(kBlock) void plan_uniform_kernel(Segment* segs, int64_t S, int n,
                                                              bool with_tree) {
    store_uniform_table(segs, S, n, with_tree);
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

// ---------------------------------------------------------------------------
// Bounds
// ---------------------------------------------------------------------------
// Work-groups of the per-tile point kernels (bounds, Morton): 16 waves per
// 4096-point tile, four points per thread.  (256 threads with 48 scalar
// loads each ran at a third of the bandwidth: too few waves per CU to cover
// the load latency.)
constexpr int kTileThreads = 1024;
constexpr int kTileRows = kSortTile / kTileThreads;

template <int D>
__global__ __launch_bounds__(kTileThreads) void bounds_kernel(const float* __restrict__ points,
                                                              const Segment* segs, int S,
                                                              float seed_lo, float seed_hi,
                                                              float* __restrict__ partials, UniformPlan plan) {
    __shared__ int s_seg;
    __shared__ float s_red[kTileThreads / kWave][2 * D];
    __shared__ float s_out[2 * D];
    const int64_t t = blockIdx.x;
    if (plan.table) store_uniform_table(plan.table, S, plan.n, plan.tree);
    int s;
    const Segment g = first_launch_segment(segs, S, plan, t, &s_seg, &s);
    const int lt = static_cast<int>(t - g.tile_first);
    if (lt >= g.tiles) return;
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);
    const PointRow<D>* rows = reinterpret_cast<const PointRow<D>*>(points + row0 * D);
    PointRow<D> r[kTileRows];
#pragma unroll
    for (int i = 0; i < kTileRows; ++i) {
        const int j = i * kTileThreads + threadIdx.x;
        if (j < count) r[i] = rows[j];
    }
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) { lo[d] = seed_lo; hi[d] = seed_hi; }
#pragma unroll
    for (int i = 0; i < kTileRows; ++i) {
        if (i * kTileThreads + static_cast<int>(threadIdx.x) < count) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                lo[d] = fminf(lo[d], r[i].v[d]);
                hi[d] = fmaxf(hi[d], r[i].v[d]);
            }
        }
    }
    block_box<D, kTileThreads>(lo, hi, s_red, s_out);
    if (threadIdx.x < 2 * D) partials[t * 2 * D + threadIdx.x] = s_out[threadIdx.x];
}

// Each cloud's bounds from its tiles' partial boxes (work-group = cloud),
// seeded with (seed_lo, seed_hi).  A separate launch rather than "last tile
// finishes": on MI355X the agent-scope release/acquire that pattern needs
// writes back and invalidates the XCD's L2 once per tile, which measured
// slower than the extra launch.
template <int D>
__global__ __launch_bounds__(kBlock) void bounds_final_kernel(const Segment* __restrict__ segs,
                                                              const float* __restrict__ partials,
                                                              float seed_lo, float seed_hi,
                                                              float* __restrict__ scene_min,
                                                              float* __restrict__ scene_max) {
    __shared__ float s_red[kBlock / kWave][2 * D];
    __shared__ float s_out[2 * D];
    const int64_t s = blockIdx.x;
    const Segment g = segs[s];
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) { lo[d] = seed_lo; hi[d] = seed_hi; }
    for (int j = threadIdx.x; j < g.tiles; j += kBlock) {
        const float* p = partials + (static_cast<int64_t>(g.tile_first) + j) * 2 * D;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            lo[d] = fminf(lo[d], p[d]);
            hi[d] = fmaxf(hi[d], p[D + d]);
        }
    }
    block_box<D>(lo, hi, s_red, s_out);
    if (threadIdx.x < D) scene_min[s * D + threadIdx.x] = s_out[threadIdx.x];
    else if (threadIdx.x < 2 * D) scene_max[s * D + threadIdx.x - D] = s_out[threadIdx.x];
}

// ---------------------------------------------------------------------------
// Primitive preparation (primitive BVH)
// ---------------------------------------------------------------------------
// One work-group per tile of 4096 primitives (V vertices of D floats):
// each primitive's vertex box and centre (sequential vertex sum / V,
// bvh_build.cu:61-93) and the tile's partial box; the cloud's bounds are
// the min of the boxes' lower corners and max of their upper corners
// (bvh_build.cu:789-791, a reduction with no seed values, so +-inf start
// it), reduced by bounds_final_kernel.
template <int D, int V>
__global__ __launch_bounds__(kBlock) void primitive_prep_kernel(const float* __restrict__ prims,
                                                                const Segment* __restrict__ segs, int S,
                                                                float* __restrict__ centers,
                                                                float* __restrict__ boxes,
                                                                float* __restrict__ partials) {
    __shared__ int s_seg;
    __shared__ float s_red[kBlock / kWave][2 * D];
    __shared__ float s_out[2 * D];
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
    for (int d = 0; d < D; ++d) { lo[d] = INFINITY; hi[d] = -INFINITY; }
    for (int j = threadIdx.x; j < count; j += kBlock) {
        const int64_t row = row0 + j;
        const float* p = prims + row * V * D;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            float b_lo = p[d], b_hi = p[d], sum = p[d];
#pragma unroll
            for (int v = 1; v < V; ++v) {
                const float x = p[v * D + d];
                b_lo = fminf(b_lo, x);
                b_hi = fmaxf(b_hi, x);
                sum += x;
            }
            centers[row * D + d] = sum / static_cast<float>(V);
            boxes[row * 2 * D + d] = b_lo;
            boxes[row * 2 * D + D + d] = b_hi;
            lo[d] = fminf(lo[d], b_lo);
            hi[d] = fmaxf(hi[d], b_hi);
        }
    }
    block_box<D>(lo, hi, s_red, s_out);
    if (threadIdx.x < 2 * D) partials[t * 2 * D + threadIdx.x] = s_out[threadIdx.x];
}

// ---------------------------------------------------------------------------
// Morton (or schedule Hilbert) keys + the first sort digit's tile counts
// ---------------------------------------------------------------------------
// One work-group per tile (the sort's tiles).  Digit counts are gathered
// with LDS atomics and stored digit-major; surplus tiles store zeros.
template <int D, bool kHilbert>
__global__ __launch_bounds__(kTileThreads) void morton_kernel(const float* __restrict__ points,
                                                              const Segment* segs, int S,
                                                              float* __restrict__ scene_min,
                                                              float* __restrict__ scene_max,
                                                              uint32_t* __restrict__ keys,
                                                              uint32_t* __restrict__ tile_hist, int64_t tstride,
                                                              int first_bit, BoundsFinish fin,
                                                              UniformPlan plan) {
    static_assert(kTileThreads >= kRadix, "one thread per digit");
    __shared__ int s_seg;
    __shared__ uint32_t s_hist[kRadix];
    __shared__ float s_red[kTileThreads / kWave][2 * D];
    __shared__ float s_box[2 * D];
    const int64_t t = blockIdx.x;
    if (threadIdx.x < kRadix) s_hist[threadIdx.x] = 0u;
    if (plan.table) store_uniform_table(plan.table, S, plan.n, plan.tree);
    int s;
    const Segment g = first_launch_segment(segs, S, plan, t, &s_seg, &s);
    const int lt = static_cast<int>(t - g.tile_first);
    if (lt >= g.tiles) {
        if (tile_hist && threadIdx.x < kRadix) tile_hist[threadIdx.x * tstride + t] = 0u;
        return;
    }
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);
    const PointRow<D>* rows = reinterpret_cast<const PointRow<D>*>(points + row0 * D);
    PointRow<D> r[kTileRows];
#pragma unroll
    for (int i = 0; i < kTileRows; ++i) {
        const int j = i * kTileThreads + threadIdx.x;
        if (j < count) r[i] = rows[j];
    }
    float lo[D], hi[D];
    if (fin.partials) {
        // The cloud's bounds from its tiles' partial boxes: every work-group
        // of the cloud reduces the same rows (min/max is exact, so all get
        // the same box) and the first one stores it.
#pragma unroll
        for (int d = 0; d < D; ++d) { lo[d] = fin.seed_lo; hi[d] = fin.seed_hi; }
        for (int j = threadIdx.x; j < g.tiles; j += kTileThreads) {
            const float* p = fin.partials + (static_cast<int64_t>(g.tile_first) + j) * 2 * D;
#pragma unroll
            for (int d = 0; d < D; ++d) {
                lo[d] = fminf(lo[d], p[d]);
                hi[d] = fmaxf(hi[d], p[D + d]);
            }
        }
        block_box<D, kTileThreads>(lo, hi, s_red, s_box);
        __syncthreads();
#pragma unroll
        for (int d = 0; d < D; ++d) {
            lo[d] = s_box[d];
            hi[d] = s_box[D + d];
        }
        if (lt == 0 && threadIdx.x < D) {
            scene_min[static_cast<int64_t>(s) * D + threadIdx.x] = s_box[threadIdx.x];
            scene_max[static_cast<int64_t>(s) * D + threadIdx.x] = s_box[D + threadIdx.x];
        }
    } else {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            lo[d] = scene_min[static_cast<int64_t>(s) * D + d];
            hi[d] = scene_max[static_cast<int64_t>(s) * D + d];
        }
    }
#pragma unroll
    for (int i = 0; i < kTileRows; ++i) {
        const int j = i * kTileThreads + threadIdx.x;
        if (j < count) {
            const uint32_t code = kHilbert ? hilbert::schedule_key<D>(r[i].v, lo, hi) : morton::encode<D>(r[i].v, lo, hi);
            keys[row0 + j] = code;
            if (tile_hist) atomicAdd(&s_hist[(code >> first_bit) & (kRadix - 1)], 1u);
        }
    }
    __syncthreads();
    if (tile_hist && threadIdx.x < kRadix) tile_hist[threadIdx.x * tstride + t] = s_hist[threadIdx.x];
}

// ---------------------------------------------------------------------------
// Implicit tree, level-synchronous passes
// ---------------------------------------------------------------------------
// Copies this group's nodes of one level (w LDS slots starting at local
// index w - 1, of which the real ones are a prefix) to their rows, which are
// contiguous in storage: every thread stores consecutive floats.
template <int D>
__device__ __forceinline__ void store_level(const float* s_box, float* nodes, int vl, int L, int lvl, int w,
                                            int gl) {
    const int j0 = gl * w;
    const int real = tree::real_at_level(vl, L, lvl) - j0;
    const int cnt = real < w ? real : w;
    if (cnt <= 0) return;
    const int64_t row0 = tree::memory_index(vl, L, tree::level_first(lvl) + j0);
    float* dst = nodes + row0 * 2 * D;
    const float* src = s_box + (w - 1) * 2 * D;
    for (int f = threadIdx.x; f < cnt * 2 * D; f += kBlock) dst[f] = src[f];
}

// Work-group `gl` of pass p owns 2^up consecutive nodes of level lvl_in
// (leaves for p == 0) and produces the `up` levels above them in LDS.  Nodes
// of a level are contiguous in storage and in LDS, so each level is stored
// by the whole group with consecutive floats per thread (one level is
// stored while the next is formed: they occupy disjoint LDS ranges).  The
// thread that forms a node writes its traversal-array entries (left/right
// child rows, leaf rank) and, for leaves, the accel's float4 point.
template <int D, bool kFromPoints>
__global__ __launch_bounds__(kBlock) void tree_pass_kernel(const float* __restrict__ points,
                                                           const Segment* __restrict__ segs, int S,
                                                           const int64_t* __restrict__ sorted,
                                                           float* __restrict__ node_aabbs, int p,
                                                           TreeOutputs out) {
    __shared__ int s_seg;
    __shared__ float s_box[(2 * kSubtreeLeaves - 1) * 2 * D];
    __shared__ uint32_t s_codes[kFromPoints ? kSubtreeLeaves + 2 * kCodeHalo : 1];
    __shared__ uint32_t s_span;
    const int64_t grp = blockIdx.x;
    if (threadIdx.x == 0) s_span = 0u;
    const int s = block_find_segment([&](int i) { return static_cast<int64_t>(segs[i].group_first[p]); },
                                     S, grp, &s_seg);
    const Segment g = segs[s];
    // The pass-indexed fields come from the table itself: indexing the local
    // copy with the runtime pass number would put the whole copy in scratch.
    const int gl = static_cast<int>(grp - segs[s].group_first[p]);
    if (gl >= segs[s].groups[p]) return;
    const int L = g.leaf_level;
    const int vl = g.vl;
    const int lvl_in = L - p * kSubtreeLevels;
    const int up = lvl_in > kSubtreeLevels ? kSubtreeLevels : lvl_in;
    const int width = 1 << up;
    float* nodes = node_aabbs + g.node_start * 2 * D;
    const bool arrays = out.left != nullptr && (out.arrays_packed || s == 0);
    const int64_t arr0 = out.arrays_packed ? g.node_start : 0;
    const int tid = threadIdx.x;
    // Fused accel: the sorted codes around this group's leaves, in LDS.
    const bool fused_accel = kFromPoints && out.sorted_codes != nullptr;
    const int g0 = gl * width;
    const int w_lo = max(g0 - kCodeHalo, 0);
    const int w_hi = min(g0 + width + kCodeHalo, g.n);
    if (fused_accel) {
        for (int k = tid; k < w_hi - w_lo; k += kBlock) s_codes[k] = out.sorted_codes[g.start + w_lo + k];
    }

    if (tid < width) {
        const int j = gl * width + tid;
        float* dst = s_box + (width - 1 + tid) * 2 * D;
        if (j < tree::real_at_level(vl, L, lvl_in)) {
            const int heap = tree::level_first(lvl_in) + j;
            const int64_t row = tree::memory_index(vl, L, heap);
            if constexpr (kFromPoints) {
                // `sorted` is this build's own sort output, a permutation of
                // [0, n) (pass 0 synthesises the values 0..n-1 and every pass
                // moves key/value pairs bijectively, tests/test_sort_model.py),
                // so the clamp never binds; it only keeps a corrupt
                // permutation from reading outside the cloud.
                const int64_t idx = min(max(sorted[g.start + j], int64_t(0)), int64_t(g.n - 1));
                if (out.leaf_boxes) {
                    // Primitive BVH: the leaf is the primitive's box.
                    const float* box = out.leaf_boxes + (g.start + idx) * 2 * D;
#pragma unroll
                    for (int c = 0; c < 2 * D; ++c) dst[c] = box[c];
                } else {
                    const float* pt = points + (g.start + idx) * D;
#pragma unroll
                    for (int d = 0; d < D; ++d) {
                        const float v = pt[d];
                        dst[d] = v;
                        dst[D + d] = v;
                    }
                }
                if (arrays) {
                    out.left[arr0 + row] = -1;
                    out.right[arr0 + row] = -1;
                    out.leaf[arr0 + row] = j;
                }
                if (out.accel_points) {
                    float4 v;
                    v.x = dst[0];
                    v.y = dst[1];
                    v.z = D == 3 ? dst[D - 1] : 0.0f;
                    v.w = __int_as_float(static_cast<int>(idx));
                    out.accel_points[g.start + j] = v;
                }
            } else {
#pragma unroll
                for (int c = 0; c < 2 * D; ++c) dst[c] = nodes[row * 2 * D + c];
            }
        }
    }
    __syncthreads();
    for (int step = 1; step <= up; ++step) {
        // The level below, complete since the last barrier (the input level
        // of a later pass is already stored).
        if (kFromPoints || step > 1) store_level<D>(s_box, nodes, vl, L, lvl_in - step + 1, width >> (step - 1), gl);
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
                if (arrays) {
                    const int left_row = tree::memory_index(vl, L, 2 * heap + 1);
                    out.left[arr0 + row] = left_row;
                    out.right[arr0 + row] = right_real ? left_row + 1 : -1;
                    out.leaf[arr0 + row] = -1;
                }
            }
        }
        __syncthreads();
    }
    if (kFromPoints || up > 0) store_level<D>(s_box, nodes, vl, L, lvl_in - up, width >> up, gl);
    if (fused_accel) {
        // Radix-tree node i = g0 + tid of this cloud (Karras 2012).  Its
        // range stays inside the group iff the first position past the
        // group's edge in its direction shares no longer prefix with i than
        // dmin; then the search and both child boxes use only LDS (the code
        // window and the subtree).  Spanning nodes are listed, compacted in
        // the group's own record rows, for launch_accel_span.
        constexpr int R = 4 * D + 4;
        const int i = g0 + tid;
        const int64_t rec0 = g.start;  // the cloud's first record row
        bool spans = false;
        if (tid < width && i < g.n - 1) {
            CodeView cv;
            cv.codes = out.sorted_codes + g.start;
            cv.win = s_codes;
            cv.w_lo = w_lo;
            cv.w_hi = w_hi;
            cv.n = g.n;
            const uint32_t ci = cv.at(i);
            int dir, dmin;
            karras_dir(cv, i, ci, dir, dmin);
            spans = cv.prefix_len(i, ci, dir > 0 ? g0 + width : g0 - 1) > dmin;
            if (!spans) {
                int first, last, gamma;
                karras_range(cv, i, ci, dir, dmin, kSubtreeLeaves, first, last, gamma);
                if (i == 0 || last - first + 1 > accel_bucket<D>()) {
                    float* rec = out.accel_records + (rec0 + i) * R;
                    float lbox[2 * D], rbox[2 * D];
                    range_box_lds<D>(s_box, width, first - g0, gamma - g0, lbox);
                    range_box_lds<D>(s_box, width, gamma + 1 - g0, last - g0, rbox);
                    store_boxes<D>(rec, lbox, rbox);
                    link_record<D>(out.accel_records + rec0 * R, i, first, gamma, last);
                }
            }
        }
        if (spans) out.span_list[rec0 + g0 + atomicAdd(&s_span, 1u)] = static_cast<uint32_t>(i);
        __syncthreads();
        if (tid == 0) out.span_count[grp] = s_span;
    }
}

inline unsigned grid_for(int64_t items) {
    return static_cast<unsigned>((items + kBlock - 1) / kBlock);
}

// Grid for a planning launch over `items` segments: enough groups to
// stream the table, capped (the kernel is grid-stride).
inline unsigned plan_grid(int64_t items) {
    const int64_t g = (items + kBlock * 4 - 1) / (kBlock * 4);
    return static_cast<unsigned>(g < 1 ? 1 : (g > 2048 ? 2048 : g));
}

}  // namespace

hipError_t launch_plan_uniform(Segment* segs, int64_t S, int64_t n, bool tree, hipStream_t stream) {
    plan_uniform_kernel<<<plan_grid(S), kBlock, 0, stream>>>(segs, S, static_cast<int>(n), tree);
    return hipGetLastError();
}

hipError_t launch_plan_offsets(Segment* segs, const int64_t* offsets, int64_t S, bool tree,
                               int64_t* node_offsets, hipStream_t stream) {
    plan_offsets_kernel<<<1, kBlock, 0, stream>>>(segs, offsets, S, tree, node_offsets);
    return hipGetLastError();
}

hipError_t launch_bounds(const float* points, int D, const Segment* segs, int64_t S,
                         int64_t tiles, float* partials, float* scene_min, float* scene_max,
                         bool finalize, float seed_lo, float seed_hi, UniformPlan plan, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(tiles);
    const unsigned cgrid = static_cast<unsigned>(S);
    const int Si = static_cast<int>(S);
    if (D == 3) {
        bounds_kernel<3><<<grid, kTileThreads, 0, stream>>>(points, segs, Si, seed_lo, seed_hi, partials, plan);
        if (finalize) {
            bounds_final_kernel<3><<<cgrid, kBlock, 0, stream>>>(segs, partials, seed_lo, seed_hi, scene_min,
                                                                 scene_max);
        }
    } else {
        bounds_kernel<2><<<grid, kTileThreads, 0, stream>>>(points, segs, Si, seed_lo, seed_hi, partials, plan);
        if (finalize) {
            bounds_final_kernel<2><<<cgrid, kBlock, 0, stream>>>(segs, partials, seed_lo, seed_hi, scene_min,
                                                                 scene_max);
        }
    }
    return hipGetLastError();
}

hipError_t launch_primitive_prep(const float* prims, int D, int V, const Segment* segs, int64_t S,
                                 int64_t tiles, float* centers, float* boxes, float* partials,
                                 float* scene_min, float* scene_max, bool finalize, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(tiles);
    const unsigned cgrid = static_cast<unsigned>(S);
    const int Si = static_cast<int>(S);
    if (D == 3 && V == 3) {
        primitive_prep_kernel<3, 3><<<grid, kBlock, 0, stream>>>(prims, segs, Si, centers, boxes, partials);
        if (finalize) {
            bounds_final_kernel<3><<<cgrid, kBlock, 0, stream>>>(segs, partials, INFINITY, -INFINITY, scene_min,
                                                                 scene_max);
        }
    } else if (D == 2 && V == 2) {
        primitive_prep_kernel<2, 2><<<grid, kBlock, 0, stream>>>(prims, segs, Si, centers, boxes, partials);
        if (finalize) {
            bounds_final_kernel<2><<<cgrid, kBlock, 0, stream>>>(segs, partials, INFINITY, -INFINITY, scene_min,
                                                                 scene_max);
        }
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_morton(const float* points, int D, const Segment* segs, int64_t S, int64_t tiles,
                         float* scene_min, float* scene_max, uint32_t* keys, uint32_t* tile_hist,
                         int64_t tstride, SortBits bits, BoundsFinish fin, hipStream_t stream,
                         UniformPlan plan) {
    const unsigned grid = static_cast<unsigned>(tiles);
    const int Si = static_cast<int>(S);
    auto run = [&](auto kernel) {
        kernel<<<grid, kTileThreads, 0, stream>>>(points, segs, Si, scene_min, scene_max, keys, tile_hist,
                                                  tstride, bits.first_bit, fin, plan);
    };
    if (D == 3) {
        bits.hilbert ? run(morton_kernel<3, true>) : run(morton_kernel<3, false>);
    } else {
        bits.hilbert ? run(morton_kernel<2, true>) : run(morton_kernel<2, false>);
    }
    return hipGetLastError();
}

hipError_t launch_tree(const float* points, int D, const Segment* segs, int64_t S, int64_t total,
                       int64_t max_n, const int64_t* sorted, float* node_aabbs,
                       const TreeOutputs& out, hipStream_t stream) {
    // Passes needed by the deepest cloud.
    const int L = tree::leaf_level(static_cast<int>(max_n));
    const int passes = L == 0 ? 1 : (L + kSubtreeLevels - 1) / kSubtreeLevels;
    const int Si = static_cast<int>(S);
    for (int p = 0; p < passes; ++p) {
        const int64_t groups = (total >> (kSubtreeLevels * (p + 1))) + S + 1;
        const unsigned grid = static_cast<unsigned>(groups);
        if (D == 3) {
            if (p == 0) tree_pass_kernel<3, true><<<grid, kBlock, 0, stream>>>(points, segs, Si, sorted, node_aabbs, p, out);
            else tree_pass_kernel<3, false><<<grid, kBlock, 0, stream>>>(points, segs, Si, sorted, node_aabbs, p, out);
        } else {
            if (p == 0) tree_pass_kernel<2, true><<<grid, kBlock, 0, stream>>>(points, segs, Si, sorted, node_aabbs, p, out);
            else tree_pass_kernel<2, false><<<grid, kBlock, 0, stream>>>(points, segs, Si, sorted, node_aabbs, p, out);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace tbvh
