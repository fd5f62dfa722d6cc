// C ABI entry points (declared in include/torchbvh_amd.h): argument checks,
// workspace carving and launch sequencing.  No entry point allocates device
// memory or synchronises the host.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/torchbvh_amd.h"
#include "tbvh_internal.hpp"

using namespace tbvh;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return TBVH_OK;
}

int hip_fail(const char* op, hipError_t e) {
    return fail(TBVH_ERR_HIP, "%s: HIP error %d (%s)", op, static_cast<int>(e), hipGetErrorString(e));
}

#define TBVH_TRY(op, expr)                       \
    do {                                         \
        const hipError_t e_ = (expr);            \
        if (e_ != hipSuccess) return hip_fail(op, e_); \
    } while (0)

// Largest cloud the implicit-tree index math supports (heap indices of the
// 2^(L+1) - 1 slots must fit in int32).
constexpr int64_t kMaxCloud = int64_t(1) << 30;
constexpr int64_t kMaxRows = 2147483647;  // INT32_MAX

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Workspace carve-out shared by build and query sort.  Every word is
// written before it is read, so nothing is cleared.
struct Layout {
    size_t segs = 0, partials = 0, keys_a = 0, keys_b = 0, vals_a = 0, vals_b = 0;
    size_t tile_hist = 0, tile_scan = 0, centers = 0, boxes = 0, total = 0;
    int64_t tiles = 0, tstride = 0;
};

// `with_primitives` adds the primitive build's centres and leaf boxes.
Layout make_layout(int64_t S, int64_t rows, int D, bool with_partials, bool with_primitives = false) {
    Layout l;
    l.tiles = tiles_bound(rows, S);
    l.tstride = tile_stride(l.tiles);
    size_t at = 0;
    l.segs = at; at = align_up(at + static_cast<size_t>(S) * sizeof(Segment));
    l.partials = at; at = align_up(at + (with_partials ? static_cast<size_t>(l.tiles) * 2 * D * sizeof(float) : 0));
    l.keys_a = at; at = align_up(at + static_cast<size_t>(rows) * 4);
    l.keys_b = at; at = align_up(at + static_cast<size_t>(rows) * 4);
    l.vals_a = at; at = align_up(at + static_cast<size_t>(rows) * 4);
    l.vals_b = at; at = align_up(at + static_cast<size_t>(rows) * 4);
    l.tile_hist = at; at = align_up(at + static_cast<size_t>(kRadix) * l.tstride * 4);
    l.tile_scan = at; at = align_up(at + static_cast<size_t>(kRadix) * l.tstride * 4);
    const size_t prim_floats = with_primitives ? static_cast<size_t>(rows) * D : 0;
    l.centers = at; at = align_up(at + prim_floats * sizeof(float));
    l.boxes = at; at = align_up(at + 2 * prim_floats * sizeof(float));
    l.total = at;
    return l;
}

template <typename T>
T* carve(void* ws, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

SortBuffers sort_buffers(void* ws, const Layout& l) {
    SortBuffers b;
    b.keys_a = carve<uint32_t>(ws, l.keys_a);
    b.keys_b = carve<uint32_t>(ws, l.keys_b);
    b.vals_a = carve<uint32_t>(ws, l.vals_a);
    b.vals_b = carve<uint32_t>(ws, l.vals_b);
    b.tile_hist = carve<uint32_t>(ws, l.tile_hist);
    b.tile_scan = carve<uint32_t>(ws, l.tile_scan);
    b.tstride = l.tstride;
    return b;
}

// Keys of the last of four passes land in keys_a (passes alternate a->b->a).
uint32_t* last_pass_keys(const SortBuffers& b) { return b.keys_a; }

int check_dim(const char* op, int D) {
    if (D != 2 && D != 3) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: D must be 2 or 3, got %d", op, D);
    return TBVH_OK;
}

int check_batched_extent(const char* op, int64_t B, int64_t N) {
    if (B < 1 || N < 1) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: B and N must be >= 1", op);
    if (N > kMaxCloud) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: a cloud may hold at most 2^30 points", op);
    if (B > kMaxRows / N) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    return TBVH_OK;
}

int check_workspace(const char* op, void* ws, size_t have, size_t need) {
    if (have < need) {
        return fail(TBVH_ERR_WORKSPACE_TOO_SMALL, "%s: workspace holds %zu bytes, %zu required", op, have, need);
    }
    if (need > 0 && ws == nullptr) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: workspace is null", op);
    if (reinterpret_cast<uintptr_t>(ws) % kAlign != 0) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: workspace must be %zu-byte aligned", op, kAlign);
    }
    return TBVH_OK;
}

bool supported_k(int k) { return k == 4 || k == 8 || k == 16 || k == 32; }


int full_key_bits(int D) { return D == 3 ? 30 : 32; }

// Digits of a full Morton sort, and of the traversal schedule (the top 16
// bits of Hilbert keys on the same grid: two passes instead of four).
SortBits full_sort(int D) { return SortBits{0, full_key_bits(D)}; }
SortBits schedule_sort(int D) { return SortBits{full_key_bits(D) - 16, full_key_bits(D), true}; }

// Everything one build call launches, in order: plan (+ clear), bounds
// (primitive builds: boxes, centres and bounds), Morton (+ the first
// digit's tile counts), four sort passes (count, scan, scatter),
// implicit-tree passes (+ traversal arrays, + accel points) and, when
// `accel` is given, the accel's radix-tree records.  `sort_only` stops
// after the sort.
struct BuildOut {
    float* node_aabbs;
    int64_t* sorted_indices;
    float* scene_min;
    float* scene_max;
    int32_t* left;
    int32_t* right;
    int32_t* leaf;
    int64_t* node_offsets;  // ragged only
    void* accel;            // optional
    bool sort_only = false;
};

// `V` > 0: `points` holds primitives of V vertices each, and the leaves are
// their boxes; the Morton codes are the centres' against the boxes' bounds.
hipError_t run_build(const float* points, const int64_t* offsets, int64_t S, int64_t n_uniform,
                     int64_t rows, int D, const BuildOut& o, void* ws, hipStream_t stream, int V = 0) {
    const Layout l = make_layout(S, rows, D, true, V > 0);
    Segment* segs = carve<Segment>(ws, l.segs);
    const SortBuffers sb = sort_buffers(ws, l);
    const bool ragged = offsets != nullptr;
    // Equal clouds of points need no planning launch: the bounds kernel
    // computes their segments and stores the table for the later launches.
    UniformPlan plan;
    hipError_t e = hipSuccess;
    if (ragged) {
        e = launch_plan_offsets(segs, offsets, S, true, o.node_offsets, stream);
    } else if (V > 0) {
        e = launch_plan_uniform(segs, S, n_uniform, true, stream);
    } else {
        plan = UniformPlan{segs, static_cast<int>(n_uniform), true};
    }
    if (e != hipSuccess) return e;
    float* partials = carve<float>(ws, l.partials);
    const float* boxes = nullptr;
    // Bounds reduced inside the Morton kernel unless a cloud may span more
    // than kFuseBoundsTiles tiles (ragged: bounded by all rows).
    const int64_t cloud_bound = ragged ? rows : n_uniform;
    const bool fuse = (cloud_bound + kSortTile - 1) / kSortTile <= kFuseBoundsTiles;
    // The point build seeds its bounds at +-1e30 (bvh_build.cu:466-467);
    // the primitive build (the boxes' min/max, bvh_build.cu:60-93) and the
    // point ordering (points.min(1) / max(1), bvh_build.cu:731-732) do not.
    const bool seeded = V == 0 && !o.sort_only;
    const float seed_lo = seeded ? kSeedLo : INFINITY;
    const float seed_hi = seeded ? kSeedHi : -INFINITY;
    BoundsFinish fin;
    if (fuse) {
        fin.partials = partials;
        fin.seed_lo = seed_lo;
        fin.seed_hi = seed_hi;
    }
    if (V > 0) {
        float* centers = carve<float>(ws, l.centers);
        float* leaf_boxes = carve<float>(ws, l.boxes);
        if ((e = launch_primitive_prep(points, D, V, segs, S, l.tiles, centers, leaf_boxes, partials,
                                       o.scene_min, o.scene_max, !fuse, stream)) != hipSuccess) {
            return e;
        }
        points = centers;
        boxes = leaf_boxes;
    }
    const SortBits bits = full_sort(D);
    uint32_t* sorted_keys = o.accel ? last_pass_keys(sb) : nullptr;
    if (V == 0 && cloud_bound <= kSmallCloud) {
        // Small clouds: bounds, codes and the whole sort in one launch.
        if ((e = launch_small_sort(points, D, segs, S, plan, cloud_bound, o.scene_min, o.scene_max, true, seed_lo,
                                   seed_hi, bits, o.sorted_indices, sorted_keys, stream)) != hipSuccess) {
            return e;
        }
    } else {
        if (V == 0 && (e = launch_bounds(points, D, segs, S, l.tiles, partials, o.scene_min, o.scene_max, !fuse,
                                         seed_lo, seed_hi, plan, stream)) != hipSuccess) {
            return e;
        }
        if ((e = launch_morton(points, D, segs, S, l.tiles, o.scene_min, o.scene_max, sb.keys_a, sb.tile_hist,
                               sb.tstride, bits, fin, stream)) != hipSuccess) {
            return e;
        }
        if ((e = launch_sort(segs, S, l.tiles, bits, sb, o.sorted_indices, sorted_keys, stream)) != hipSuccess) {
            return e;
        }
    }
    if (o.sort_only) return hipSuccess;
    TreeOutputs to;
    to.left = o.left;
    to.right = o.right;
    to.leaf = o.leaf;
    to.arrays_packed = ragged;
    to.accel_points = o.accel ? static_cast<float4*>(o.accel) : nullptr;
    to.leaf_boxes = boxes;
    if (o.accel) {
        // Radix-tree records in the first tree pass; the sort's value
        // buffers (dead after the sort) hold the spanning-node marks.
        to.sorted_codes = sorted_keys;
        to.accel_records = reinterpret_cast<float*>(static_cast<char*>(o.accel) + accel_points_bytes(rows));
        to.span_list = sb.vals_a;
        to.span_count = sb.vals_b;
    }
    const int64_t max_n = ragged ? (rows < kMaxCloud ? rows : kMaxCloud) : n_uniform;
    if ((e = launch_tree(points, D, segs, S, rows, max_n, o.sorted_indices, o.node_aabbs, to,
                         stream)) != hipSuccess) {
        return e;
    }
    if (o.accel) {
        // First-pass work-groups: at most one per 256 leaves of each cloud.
        const int64_t groups_bound = (rows + kSubtreeLeaves - 1) / kSubtreeLeaves + S;
        return launch_accel_span(o.node_aabbs, D, segs, S, rows, groups_bound, sorted_keys, sb.vals_a, sb.vals_b,
                                 o.accel, stream);
    }
    return hipSuccess;
}

hipError_t run_query_sort(const float* queries, const int64_t* offsets, int64_t S, int64_t m_uniform,
                          int64_t rows, int D, const float* scene_min, const float* scene_max,
                          SortBits bits, int64_t* order, uint32_t* codes_only, void* ws,
                          hipStream_t stream) {
    const Layout l = make_layout(S, rows, D, false);
    Segment* segs = carve<Segment>(ws, l.segs);
    const SortBuffers sb = sort_buffers(ws, l);
    // Equal clouds need no planning launch: the Morton kernel computes their
    // segments and stores the table for the sort.
    UniformPlan plan;
    hipError_t e = hipSuccess;
    if (offsets) e = launch_plan_offsets(segs, offsets, S, false, nullptr, stream);
    else plan = UniformPlan{segs, static_cast<int>(m_uniform), false};
    if (e != hipSuccess) return e;
    const int64_t m_bound = offsets ? rows : m_uniform;  // bounds every cloud's query count
    if (!codes_only && m_bound >= 1 && m_bound <= kSmallCloud) {
        // Small query sets: codes and the whole sort in one launch.
        return launch_small_sort(queries, D, segs, S, plan, m_bound, const_cast<float*>(scene_min),
                                 const_cast<float*>(scene_max), false, 0.0f, 0.0f, bits, order, nullptr, stream);
    }
    uint32_t* keys = codes_only ? codes_only : sb.keys_a;
    // Bounds given (BoundsFinish empty): the kernel only reads them.
    if ((e = launch_morton(queries, D, segs, S, l.tiles, const_cast<float*>(scene_min),
                           const_cast<float*>(scene_max), keys, codes_only ? nullptr : sb.tile_hist, sb.tstride,
                           bits, BoundsFinish{}, stream, plan)) != hipSuccess) {
        return e;
    }
    if (codes_only) return hipSuccess;
    return launch_sort(segs, S, l.tiles, bits, sb, order, nullptr, stream);
}

bool aligned(const void* p) { return reinterpret_cast<uintptr_t>(p) % kAlign == 0; }

}  // namespace

extern "C" {

int tbvh_abi_version(void) { return TBVH_ABI_VERSION; }

const char* tbvh_last_error(void) { return g_last_error.c_str(); }

int tbvh_leaf_level(int64_t n) {
    if (n < 1 || n > kMaxCloud) return -1;
    return tree::leaf_level(static_cast<int>(n));
}

int64_t tbvh_virtual_leaves(int64_t n) {
    if (n < 1 || n > kMaxCloud) return -1;
    return tree::virtual_leaves(static_cast<int>(n));
}

int64_t tbvh_real_node_count(int64_t n) {
    if (n < 1 || n > kMaxCloud) return -1;
    return tree::real_node_count(static_cast<int>(n));
}

// ---------------------------------------------------------------------------
// Build
// ---------------------------------------------------------------------------
int tbvh_build_workspace_size(int64_t B, int64_t N, int D, size_t* bytes) {
    const char* op = "tbvh_build_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    *bytes = make_layout(B, B * N, D, true).total;
    return ok();
}

static int build_batched(const char* op, const float* points, int64_t B, int64_t N, int D,
                         const BuildOut& o, void* workspace, size_t workspace_bytes,
                         void* stream_ptr) {
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    if (!points || !o.node_aabbs || !o.sorted_indices || !o.scene_min || !o.scene_max || !o.left ||
        !o.right || !o.leaf) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (o.accel) {
        if (N > kMaxAccelCloud) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: clouds may hold at most 2^28 points", op);
        if (!aligned(o.accel)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    }
    const Layout l = make_layout(B, B * N, D, true);
    if (int r = check_workspace(op, workspace, workspace_bytes, l.total)) return r;
    TBVH_TRY(op, run_build(points, nullptr, B, N, B * N, D, o, workspace,
                           static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_build(const float* points, int64_t B, int64_t N, int D, float* node_aabbs,
               int64_t* sorted_indices, float* scene_min, float* scene_max,
               int32_t* left_child_mem, int32_t* right_child_mem, int32_t* mem_to_leaf,
               void* workspace, size_t workspace_bytes, void* stream_ptr) {
    const BuildOut o{node_aabbs, sorted_indices, scene_min, scene_max, left_child_mem,
                     right_child_mem, mem_to_leaf, nullptr, nullptr};
    return build_batched("tbvh_build", points, B, N, D, o, workspace, workspace_bytes, stream_ptr);
}

int tbvh_build_with_accel(const float* points, int64_t B, int64_t N, int D, float* node_aabbs,
                          int64_t* sorted_indices, float* scene_min, float* scene_max,
                          int32_t* left_child_mem, int32_t* right_child_mem, int32_t* mem_to_leaf,
                          void* accel, void* workspace, size_t workspace_bytes, void* stream_ptr) {
    if (!accel) return fail(TBVH_ERR_INVALID_ARGUMENT, "tbvh_build_with_accel: accel is null");
    const BuildOut o{node_aabbs, sorted_indices, scene_min, scene_max, left_child_mem,
                     right_child_mem, mem_to_leaf, nullptr, accel};
    return build_batched("tbvh_build_with_accel", points, B, N, D, o, workspace, workspace_bytes,
                         stream_ptr);
}

}  // extern "C"

// Workspace of tbvh_build_with_accel_noalloc: one array per GPU, in each
// GPU's copy of this code object.  In host code `noalloc_scratch` names a
// host-side stand-in, never the device memory: only the addresses that
// hipGetSymbolAddress returns (kept per device) are passed to kernels.
namespace {

static __device__ __align__(256) unsigned char noalloc_scratch[TBVH_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 256;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// Device address of the current device's array, looked up once per device
// with that device current.
int noalloc_scratch_for(const char* op, hipStream_t stream, void** out) {
    int dev = -1;
    TBVH_TRY(op, hipGetDevice(&dev));
    int stream_dev = -1;
    TBVH_TRY(op, hipStreamGetDevice(stream, &stream_dev));
    if (stream_dev != dev) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: the stream belongs to device %d, but device %d is current",
                    op, stream_dev, dev);
    }
    if (dev < 0 || dev >= kMaxDevices) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: device %d out of range", op, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        TBVH_TRY(op, hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch)));
        if (p == nullptr || reinterpret_cast<uintptr_t>(p) % kAlign != 0) {
            return fail(TBVH_ERR_HIP, "%s: the scratch array has no usable device address", op);
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return TBVH_OK;
}

}  // namespace

extern "C" {

int tbvh_build_with_accel_noalloc(const float* points, int64_t B, int64_t N, int D, float* node_aabbs,
                                  int64_t* sorted_indices, float* scene_min, float* scene_max,
                                  int32_t* left_child_mem, int32_t* right_child_mem, int32_t* mem_to_leaf,
                                  void* accel, void* stream_ptr) {
    const char* op = "tbvh_build_with_accel_noalloc";
    if (!accel) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel is null", op);
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    const size_t need = make_layout(B, B * N, D, true).total;
    if (need > TBVH_NOALLOC_SCRATCH_BYTES) {
        return fail(TBVH_ERR_WORKSPACE_TOO_SMALL,
                    "%s: %lld x %lld points need %zu bytes of workspace; the library's scratch array holds %zu",
                    op, static_cast<long long>(B), static_cast<long long>(N), need,
                    static_cast<size_t>(TBVH_NOALLOC_SCRATCH_BYTES));
    }
    void* scratch = nullptr;
    if (int r = noalloc_scratch_for(op, static_cast<hipStream_t>(stream_ptr), &scratch)) return r;
    const BuildOut o{node_aabbs, sorted_indices, scene_min, scene_max, left_child_mem,
                     right_child_mem, mem_to_leaf, nullptr, accel};
    return build_batched(op, points, B, N, D, o, scratch, TBVH_NOALLOC_SCRATCH_BYTES, stream_ptr);
}

int tbvh_build_ragged_workspace_size(int64_t B, int64_t total, int D, size_t* bytes) {
    const char* op = "tbvh_build_ragged_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || total < B) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total >= B", op);
    if (total > kMaxRows) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    *bytes = make_layout(B, total, D, true).total;
    return ok();
}

static int build_ragged(const char* op, const float* points, const int64_t* offsets, int64_t B,
                        int64_t total, int D, const BuildOut& o, int64_t total_nodes,
                        void* workspace, size_t workspace_bytes, void* stream_ptr) {
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || total < B) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total >= B", op);
    if (total > kMaxRows) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    if (total_nodes < 2 * total - B) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total_nodes is smaller than any tree over %lld points",
                    op, static_cast<long long>(total));
    }
    if (!points || !offsets || !o.node_aabbs || !o.sorted_indices || !o.scene_min || !o.scene_max ||
        !o.left || !o.right || !o.leaf || !o.node_offsets) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (o.accel && !aligned(o.accel)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    }
    const Layout l = make_layout(B, total, D, true);
    if (int r = check_workspace(op, workspace, workspace_bytes, l.total)) return r;
    TBVH_TRY(op, run_build(points, offsets, B, 0, total, D, o, workspace,
                           static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_build_ragged(const float* points, const int64_t* offsets, int64_t B, int64_t total, int D,
                      float* node_aabbs, int64_t* sorted_indices, float* scene_min,
                      float* scene_max, int32_t* left_child_mem, int32_t* right_child_mem,
                      int32_t* mem_to_leaf, int64_t* node_offsets, int64_t total_nodes,
                      void* workspace, size_t workspace_bytes, void* stream_ptr) {
    const BuildOut o{node_aabbs, sorted_indices, scene_min, scene_max, left_child_mem,
                     right_child_mem, mem_to_leaf, node_offsets, nullptr};
    return build_ragged("tbvh_build_ragged", points, offsets, B, total, D, o, total_nodes, workspace,
                        workspace_bytes, stream_ptr);
}

int tbvh_build_ragged_with_accel(const float* points, const int64_t* offsets, int64_t B,
                                 int64_t total, int D, float* node_aabbs, int64_t* sorted_indices,
                                 float* scene_min, float* scene_max, int32_t* left_child_mem,
                                 int32_t* right_child_mem, int32_t* mem_to_leaf,
                                 int64_t* node_offsets, int64_t total_nodes, void* accel,
                                 void* workspace, size_t workspace_bytes, void* stream_ptr) {
    if (!accel) return fail(TBVH_ERR_INVALID_ARGUMENT, "tbvh_build_ragged_with_accel: accel is null");
    if (total > kMaxAccelCloud * B) {
        // A cheap necessary condition; the caller checks each cloud's size.
        return fail(TBVH_ERR_INVALID_ARGUMENT, "tbvh_build_ragged_with_accel: clouds may hold at most 2^28 points");
    }
    const BuildOut o{node_aabbs, sorted_indices, scene_min, scene_max, left_child_mem,
                     right_child_mem, mem_to_leaf, node_offsets, accel};
    return build_ragged("tbvh_build_ragged_with_accel", points, offsets, B, total, D, o, total_nodes,
                        workspace, workspace_bytes, stream_ptr);
}

// ---------------------------------------------------------------------------
// Primitive build and point ordering
// ---------------------------------------------------------------------------
static int check_primitive_shape(const char* op, int64_t B, int64_t F, int V, int D) {
    if (!((V == 2 && D == 2) || (V == 3 && D == 3))) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: expected 2-D segments or 3-D triangles", op);
    }
    return check_batched_extent(op, B, F);
}

int tbvh_build_primitives_workspace_size(int64_t B, int64_t F, int V, int D, size_t* bytes) {
    const char* op = "tbvh_build_primitives_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_primitive_shape(op, B, F, V, D)) return r;
    *bytes = make_layout(B, B * F, D, true, true).total;
    return ok();
}

int tbvh_build_primitives(const float* primitives, int64_t B, int64_t F, int V, int D, float* node_aabbs,
                          int64_t* sorted_indices, float* scene_min, float* scene_max,
                          int32_t* left_child_mem, int32_t* right_child_mem, int32_t* mem_to_leaf,
                          void* workspace, size_t workspace_bytes, void* stream_ptr) {
    const char* op = "tbvh_build_primitives";
    if (int r = check_primitive_shape(op, B, F, V, D)) return r;
    if (!primitives || !node_aabbs || !sorted_indices || !scene_min || !scene_max || !left_child_mem ||
        !right_child_mem || !mem_to_leaf) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    const Layout l = make_layout(B, B * F, D, true, true);
    if (int r = check_workspace(op, workspace, workspace_bytes, l.total)) return r;
    const BuildOut o{node_aabbs, sorted_indices, scene_min, scene_max, left_child_mem,
                     right_child_mem, mem_to_leaf, nullptr, nullptr};
    TBVH_TRY(op, run_build(primitives, nullptr, B, F, B * F, D, o, workspace,
                           static_cast<hipStream_t>(stream_ptr), V));
    return ok();
}

// The point ordering needs the clouds' bounds only in the workspace: they
// sit after the build layout.
static size_t point_sort_bytes(int64_t B, int64_t N, int D, size_t* bounds_at) {
    const size_t at = make_layout(B, B * N, D, true).total;
    if (bounds_at) *bounds_at = at;
    return at + align_up(2 * static_cast<size_t>(B) * D * sizeof(float));
}

int tbvh_morton_sort_points_workspace_size(int64_t B, int64_t N, int D, size_t* bytes) {
    const char* op = "tbvh_morton_sort_points_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    *bytes = point_sort_bytes(B, N, D, nullptr);
    return ok();
}

int tbvh_morton_sort_points(const float* points, int64_t B, int64_t N, int D, int64_t* sorted_indices,
                            void* workspace, size_t workspace_bytes, void* stream_ptr) {
    const char* op = "tbvh_morton_sort_points";
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    if (!points || !sorted_indices) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    size_t bounds_at = 0;
    if (int r = check_workspace(op, workspace, workspace_bytes, point_sort_bytes(B, N, D, &bounds_at))) return r;
    float* scene_min = carve<float>(workspace, bounds_at);
    float* scene_max = scene_min + B * D;
    BuildOut o{nullptr, sorted_indices, scene_min, scene_max, nullptr, nullptr, nullptr, nullptr, nullptr};
    o.sort_only = true;
    TBVH_TRY(op, run_build(points, nullptr, B, N, B * N, D, o, workspace,
                           static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

// ---------------------------------------------------------------------------
// Query ordering
// ---------------------------------------------------------------------------
int tbvh_sort_queries_workspace_size(int64_t B, int64_t M, int D, size_t* bytes) {
    const char* op = "tbvh_sort_queries_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    *bytes = make_layout(B, B * M, D, false).total;
    return ok();
}

static int sort_batched(const char* op, const float* queries, int64_t B, int64_t M, int D,
                        const float* scene_min, const float* scene_max, bool schedule, int64_t* order,
                        uint32_t* codes, void* workspace, size_t workspace_bytes, void* stream_ptr) {
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (M == 0) return ok();
    if (M > kMaxCloud) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: at most 2^30 queries per cloud", op);
    if (!queries || !scene_min || !scene_max || (!order && !codes)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    const Layout l = make_layout(B, B * M, D, false);
    if (int r = check_workspace(op, workspace, workspace_bytes, l.total)) return r;
    TBVH_TRY(op, run_query_sort(queries, nullptr, B, M, B * M, D, scene_min, scene_max,
                                schedule ? schedule_sort(D) : full_sort(D), order, codes, workspace,
                                static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_sort_queries(const float* queries, int64_t B, int64_t M, int D, const float* scene_min,
                      const float* scene_max, int64_t* order, void* workspace,
                      size_t workspace_bytes, void* stream_ptr) {
    if (!order && M > 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "tbvh_sort_queries: null input or output pointer");
    return sort_batched("tbvh_sort_queries", queries, B, M, D, scene_min, scene_max, false, order,
                        nullptr, workspace, workspace_bytes, stream_ptr);
}

int tbvh_schedule_queries(const float* queries, int64_t B, int64_t M, int D, const float* scene_min,
                          const float* scene_max, int64_t* order, void* workspace,
                          size_t workspace_bytes, void* stream_ptr) {
    if (!order && M > 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "tbvh_schedule_queries: null input or output pointer");
    return sort_batched("tbvh_schedule_queries", queries, B, M, D, scene_min, scene_max, true, order,
                        nullptr, workspace, workspace_bytes, stream_ptr);
}

int tbvh_morton_codes(const float* rows, int64_t B, int64_t M, int D, const float* scene_min,
                      const float* scene_max, uint32_t* codes, void* workspace,
                      size_t workspace_bytes, void* stream_ptr) {
    if (!codes && M > 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "tbvh_morton_codes: null input or output pointer");
    return sort_batched("tbvh_morton_codes", rows, B, M, D, scene_min, scene_max, false, nullptr, codes,
                        workspace, workspace_bytes, stream_ptr);
}

int tbvh_sort_queries_ragged_workspace_size(int64_t B, int64_t total_q, int D, size_t* bytes) {
    const char* op = "tbvh_sort_queries_ragged_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || total_q < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total_q >= 0", op);
    if (total_q > kMaxRows) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    *bytes = make_layout(B, total_q, D, false).total;
    return ok();
}

static int sort_ragged(const char* op, const float* queries, const int64_t* query_offsets, int64_t B,
                       int64_t total_q, int D, const float* scene_min, const float* scene_max,
                       bool schedule, int64_t* order, void* workspace, size_t workspace_bytes,
                       void* stream_ptr) {
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || total_q < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total_q >= 0", op);
    if (total_q > kMaxRows) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (total_q == 0) return ok();
    if (!queries || !query_offsets || !scene_min || !scene_max || !order) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    const Layout l = make_layout(B, total_q, D, false);
    if (int r = check_workspace(op, workspace, workspace_bytes, l.total)) return r;
    TBVH_TRY(op, run_query_sort(queries, query_offsets, B, 0, total_q, D, scene_min, scene_max,
                                schedule ? schedule_sort(D) : full_sort(D), order, nullptr, workspace,
                                static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_sort_queries_ragged(const float* queries, const int64_t* query_offsets, int64_t B,
                             int64_t total_q, int D, const float* scene_min,
                             const float* scene_max, int64_t* order, void* workspace,
                             size_t workspace_bytes, void* stream_ptr) {
    return sort_ragged("tbvh_sort_queries_ragged", queries, query_offsets, B, total_q, D, scene_min,
                       scene_max, false, order, workspace, workspace_bytes, stream_ptr);
}

int tbvh_schedule_queries_ragged(const float* queries, const int64_t* query_offsets, int64_t B,
                                 int64_t total_q, int D, const float* scene_min,
                                 const float* scene_max, int64_t* order, void* workspace,
                                 size_t workspace_bytes, void* stream_ptr) {
    return sort_ragged("tbvh_schedule_queries_ragged", queries, query_offsets, B, total_q, D,
                       scene_min, scene_max, true, order, workspace, workspace_bytes, stream_ptr);
}

// ---------------------------------------------------------------------------
// Routed query ordering
// ---------------------------------------------------------------------------
namespace {

struct RoutedLayout {
    size_t part, gathered, offsets, gmin, gmax, sorted_local, total;
};

RoutedLayout make_routed_layout(int64_t B, int64_t M, int D) {
    const int64_t rows = B * M;
    const size_t sort_a = make_layout(B, rows, D, false).total;
    const size_t sort_b = make_layout(2 * B, rows, D, false).total;
    RoutedLayout r;
    size_t at = align_up(sort_a > sort_b ? sort_a : sort_b);
    r.part = at; at = align_up(at + static_cast<size_t>(rows) * 8);
    r.gathered = at; at = align_up(at + static_cast<size_t>(rows) * D * 4);
    r.offsets = at; at = align_up(at + static_cast<size_t>(2 * B + 1) * 8);
    r.gmin = at; at = align_up(at + static_cast<size_t>(2 * B) * D * 4);
    r.gmax = at; at = align_up(at + static_cast<size_t>(2 * B) * D * 4);
    r.sorted_local = at; at = align_up(at + static_cast<size_t>(rows) * 8);
    r.total = at;
    return r;
}

hipError_t run_routed_sort(const float* queries, const uint8_t* routes, int64_t B, int64_t M, int D,
                           const float* true_min, const float* true_max, const float* false_min,
                           const float* false_max, int64_t* order, void* ws, hipStream_t stream) {
    const int64_t rows = B * M;
    const RoutedLayout r = make_routed_layout(B, M, D);
    int64_t* part = carve<int64_t>(ws, r.part);
    float* gathered = carve<float>(ws, r.gathered);
    int64_t* group_offsets = carve<int64_t>(ws, r.offsets);
    float* gmin = carve<float>(ws, r.gmin);
    float* gmax = carve<float>(ws, r.gmax);
    int64_t* sorted_local = carve<int64_t>(ws, r.sorted_local);
    // 1. Stable partition of every cloud by route (one 8-bit pass on 0/1).
    const Layout l = make_layout(B, rows, D, false);
    Segment* segs = carve<Segment>(ws, l.segs);
    const SortBuffers sb = sort_buffers(ws, l);
    hipError_t e = launch_plan_uniform(segs, B, M, false, stream);
    if (e != hipSuccess) return e;
    if ((e = launch_route_keys(routes, segs, B, l.tiles, sb.keys_a, sb.tile_hist, sb.tstride, stream)) !=
        hipSuccess) {
        return e;
    }
    if ((e = launch_sort(segs, B, l.tiles, SortBits{0, kRadixBits}, sb, part, nullptr, stream)) != hipSuccess) {
        return e;
    }
    // 2. Partitioned queries as 2B segments (false group, true group per cloud).
    if ((e = launch_route_gather(queries, part, segs, sb.tile_scan, B, M, D, true_min, true_max, false_min, false_max,
                                 gathered, group_offsets, gmin, gmax, stream)) != hipSuccess) {
        return e;
    }
    // 3. Morton order within every group, against the group's route bounds.
    if ((e = run_query_sort(gathered, group_offsets, 2 * B, 0, rows, D, gmin, gmax, full_sort(D), sorted_local,
                            nullptr, ws, stream)) != hipSuccess) {
        return e;
    }
    // 4. Back to query indices.
    return launch_route_finish(part, sorted_local, group_offsets, B, M, order, stream);
}

}  // namespace

int tbvh_sort_routed_queries_workspace_size(int64_t B, int64_t M, int D, size_t* bytes) {
    const char* op = "tbvh_sort_routed_queries_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    *bytes = make_routed_layout(B, M, D).total;
    return ok();
}

int tbvh_sort_routed_queries(const float* queries, const uint8_t* routes, int64_t B, int64_t M, int D,
                             const float* true_min, const float* true_max, const float* false_min,
                             const float* false_max, int64_t* order, void* workspace,
                             size_t workspace_bytes, void* stream_ptr) {
    const char* op = "tbvh_sort_routed_queries";
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (M == 0) return ok();
    if (M > kMaxCloud) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: at most 2^30 queries per cloud", op);
    if (!queries || !routes || !true_min || !true_max || !false_min || !false_max || !order) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (int r = check_workspace(op, workspace, workspace_bytes, make_routed_layout(B, M, D).total)) return r;
    TBVH_TRY(op, run_routed_sort(queries, routes, B, M, D, true_min, true_max, false_min, false_max, order,
                                 workspace, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

// ---------------------------------------------------------------------------
// k-NN
// ---------------------------------------------------------------------------
static int knn_batched(const char* op, const float* node_aabbs, const int64_t* sorted_indices,
                       const float* queries, const int64_t* order, int64_t B, int64_t M,
                       int64_t num_leaves, int64_t num_real_nodes, int D, int k, bool spatial,
                       int64_t* out_indices, float* out_distances, void* stream_ptr) {
    if (int r = check_dim(op, D)) return r;
    if (!supported_k(k)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: k must be 4, 8, or 16 (32 is also supported), got %d", op, k);
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (num_leaves < 1 || num_leaves > kMaxCloud) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_leaves must be in [1, 2^30]", op);
    }
    if (num_leaves < k) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_leaves must be >= k", op);
    if (num_real_nodes != tree::real_node_count(static_cast<int>(num_leaves))) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_real_nodes does not match num_leaves", op);
    }
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (B > kMaxRows / num_leaves) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    if (M == 0) return ok();
    if (!node_aabbs || !sorted_indices || !queries || !out_indices || !out_distances || (spatial && !order)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    KnnArgs a{};
    a.node_aabbs = node_aabbs;
    a.sorted_indices = sorted_indices;
    a.queries = queries;
    a.order = order;
    a.B = B;
    a.M = M;
    a.total_q = B * M;
    a.num_leaves = static_cast<int32_t>(num_leaves);
    a.num_real_nodes = static_cast<int32_t>(num_real_nodes);
    a.out_indices = out_indices;
    a.out_distances = out_distances;
    a.spatial_output = spatial;
    TBVH_TRY(op, launch_knn(a, D, k, false, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_knn(const float* node_aabbs, const int64_t* sorted_indices, const float* queries,
             const int64_t* order, int64_t B, int64_t M, int64_t num_leaves,
             int64_t num_real_nodes, int D, int k, int64_t* out_indices, float* out_distances,
             void* stream_ptr) {
    return knn_batched("tbvh_knn", node_aabbs, sorted_indices, queries, order, B, M, num_leaves,
                       num_real_nodes, D, k, false, out_indices, out_distances, stream_ptr);
}

int tbvh_knn_spatial(const float* node_aabbs, const int64_t* sorted_indices, const float* queries,
                     const int64_t* order, int64_t B, int64_t M, int64_t num_leaves,
                     int64_t num_real_nodes, int D, int k, int64_t* out_indices,
                     float* out_distances, void* stream_ptr) {
    return knn_batched("tbvh_knn_spatial", node_aabbs, sorted_indices, queries, order, B, M,
                       num_leaves, num_real_nodes, D, k, true, out_indices, out_distances,
                       stream_ptr);
}

int tbvh_knn_ragged(const float* node_aabbs, const int64_t* sorted_indices,
                    const int64_t* point_offsets, const int64_t* node_offsets,
                    const float* queries, const int64_t* query_offsets, const int64_t* order,
                    int64_t B, int64_t total_q, int D, int k, int64_t* out_indices,
                    float* out_distances, void* stream_ptr) {
    const char* op = "tbvh_knn_ragged";
    if (int r = check_dim(op, D)) return r;
    if (!supported_k(k)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: k must be 4, 8, or 16 (32 is also supported), got %d", op, k);
    if (B < 1 || total_q < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total_q >= 0", op);
    if (total_q > kMaxRows) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (total_q == 0) return ok();
    if (!node_aabbs || !sorted_indices || !point_offsets || !node_offsets || !queries ||
        !query_offsets || !out_indices || !out_distances) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    KnnArgs a{};
    a.node_aabbs = node_aabbs;
    a.sorted_indices = sorted_indices;
    a.queries = queries;
    a.order = order;
    a.point_offsets = point_offsets;
    a.node_offsets = node_offsets;
    a.query_offsets = query_offsets;
    a.B = B;
    a.total_q = total_q;
    a.out_indices = out_indices;
    a.out_distances = out_distances;
    TBVH_TRY(op, launch_knn(a, D, k, true, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

// ---------------------------------------------------------------------------
// Acceleration structure
// ---------------------------------------------------------------------------
namespace {

size_t accel_workspace_bytes(int64_t S, int64_t total) {
    return align_up(static_cast<size_t>(S) * sizeof(Segment)) + align_up(static_cast<size_t>(total) * 4);
}

int check_accel_extent(const char* op, int64_t B, int64_t total, int D) {
    if (int r = check_dim(op, D)) return r;
    if (B < 1 || total < B) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total >= B", op);
    if (total > kMaxRows) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    return TBVH_OK;
}

}  // namespace

int tbvh_accel_size(int64_t B, int64_t total_points, int D, size_t* bytes) {
    const char* op = "tbvh_accel_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_accel_extent(op, B, total_points, D)) return r;
    *bytes = accel_bytes(total_points, B, D);
    return ok();
}

int tbvh_accel_workspace_size(int64_t B, int64_t total_points, int D, size_t* bytes) {
    const char* op = "tbvh_accel_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: bytes is null", op);
    if (int r = check_accel_extent(op, B, total_points, D)) return r;
    *bytes = accel_workspace_bytes(B, total_points);
    return ok();
}

int tbvh_accel_build(const float* points, const int64_t* sorted_indices, const float* node_aabbs,
                     const float* scene_min, const float* scene_max, int64_t B, int64_t N, int D,
                     void* accel, void* workspace, size_t workspace_bytes, void* stream_ptr) {
    const char* op = "tbvh_accel_build";
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    if (N > kMaxAccelCloud) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: clouds may hold at most 2^28 points", op);
    if (!points || !sorted_indices || !node_aabbs || !scene_min || !scene_max || !accel) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    const int64_t total = B * N;
    if (int r = check_workspace(op, workspace, workspace_bytes, accel_workspace_bytes(B, total))) return r;
    if (reinterpret_cast<uintptr_t>(accel) % kAlign != 0) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    Segment* segs = carve<Segment>(workspace, 0);
    uint32_t* codes = carve<uint32_t>(workspace, align_up(static_cast<size_t>(B) * sizeof(Segment)));
    TBVH_TRY(op, launch_plan_uniform(segs, B, N, true, stream));
    TBVH_TRY(op, launch_accel_points(points, sorted_indices, scene_min, scene_max, D, segs, B, total,
                                     codes, accel, stream));
    TBVH_TRY(op, launch_accel_nodes(node_aabbs, D, segs, B, total, codes, accel, stream));
    return ok();
}

int tbvh_accel_build_from_tree(const float* node_aabbs, const int64_t* sorted_indices, int64_t B, int64_t N,
                               int64_t num_real_nodes, int D, void* accel, uint32_t* defects, void* workspace,
                               size_t workspace_bytes, void* stream_ptr) {
    const char* op = "tbvh_accel_build_from_tree";
    if (int r = check_dim(op, D)) return r;
    if (int r = check_batched_extent(op, B, N)) return r;
    if (N > kMaxAccelCloud) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: clouds may hold at most 2^28 points", op);
    if (num_real_nodes != tree::real_node_count(static_cast<int>(N))) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_real_nodes does not match num_leaves", op);
    }
    if (!node_aabbs || !sorted_indices || !accel || !defects) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    const int64_t total = B * N;
    if (int r = check_workspace(op, workspace, workspace_bytes, accel_workspace_bytes(B, total))) return r;
    if (reinterpret_cast<uintptr_t>(accel) % kAlign != 0) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    Segment* segs = carve<Segment>(workspace, 0);
    uint32_t* codes = carve<uint32_t>(workspace, align_up(static_cast<size_t>(B) * sizeof(Segment)));
    TBVH_TRY(op, launch_tree_defects(node_aabbs, sorted_indices, D, B, static_cast<int>(N),
                                     static_cast<int>(num_real_nodes), defects, stream));
    TBVH_TRY(op, launch_plan_uniform(segs, B, N, true, stream));
    TBVH_TRY(op, launch_accel_points_from_tree(node_aabbs, sorted_indices, D, segs, B, total, codes, accel, stream));
    TBVH_TRY(op, launch_accel_nodes(node_aabbs, D, segs, B, total, codes, accel, stream));
    return ok();
}

int tbvh_accel_build_ragged(const float* points, const int64_t* offsets, const int64_t* sorted_indices,
                            const float* node_aabbs, const float* scene_min, const float* scene_max,
                            int64_t B, int64_t total, int D, void* accel, void* workspace,
                            size_t workspace_bytes, void* stream_ptr) {
    const char* op = "tbvh_accel_build_ragged";
    if (int r = check_accel_extent(op, B, total, D)) return r;
    if (!points || !offsets || !sorted_indices || !node_aabbs || !scene_min || !scene_max || !accel) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (int r = check_workspace(op, workspace, workspace_bytes, accel_workspace_bytes(B, total))) return r;
    if (reinterpret_cast<uintptr_t>(accel) % kAlign != 0) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    }
    hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    Segment* segs = carve<Segment>(workspace, 0);
    uint32_t* codes = carve<uint32_t>(workspace, align_up(static_cast<size_t>(B) * sizeof(Segment)));
    TBVH_TRY(op, launch_plan_offsets(segs, offsets, B, true, nullptr, stream));
    TBVH_TRY(op, launch_accel_points(points, sorted_indices, scene_min, scene_max, D, segs, B, total,
                                     codes, accel, stream));
    TBVH_TRY(op, launch_accel_nodes(node_aabbs, D, segs, B, total, codes, accel, stream));
    return ok();
}

static int knn_accel_batched(const char* op, const void* accel, const float* queries,
                             const int64_t* order, int64_t B, int64_t M, int64_t num_leaves, int D,
                             int k, bool spatial, int64_t* out_indices, float* out_distances,
                             void* stream_ptr, const float* source_points = nullptr, int source_cols = 0,
                             float* out_positions = nullptr, const float* node_aabbs = nullptr,
                             int64_t num_real_nodes = 0, void* ws = nullptr, size_t ws_bytes = 0) {
    if (int r = check_dim(op, D)) return r;
    if (!supported_k(k)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: k must be 4, 8, or 16 (32 is also supported), got %d", op, k);
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (num_leaves < 1 || num_leaves > kMaxAccelCloud) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_leaves must be in [1, 2^28]", op);
    }
    if (num_leaves < k) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_leaves must be >= k", op);
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (B > kMaxRows / num_leaves) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    if (M == 0) return ok();
    if (!accel || !queries || !out_indices || !out_distances || (spatial && !order)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (!aligned(accel)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    KnnArgs a{};
    a.queries = queries;
    a.order = order;
    a.B = B;
    a.M = M;
    a.total_q = B * M;
    a.num_leaves = static_cast<int32_t>(num_leaves);
    a.out_indices = out_indices;
    a.out_distances = out_distances;
    a.accel = accel;
    a.total_points = B * num_leaves;
    a.spatial_output = spatial;
    a.source_points = source_points;
    a.source_cols = source_cols;
    a.out_positions = out_positions;
    const int level = ws ? grid_level(num_leaves, D, k) : 0;
    if (level > 0) {
        if (!node_aabbs) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null node_aabbs", op);
        if (num_real_nodes != tree::real_node_count(static_cast<int>(num_leaves))) {
            return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_real_nodes does not match num_leaves", op);
        }
        if (!aligned(ws)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: workspace must be %zu-byte aligned", op, kAlign);
        const size_t need = grid_workspace_bytes(B, B * M, level, D);
        if (ws_bytes < need) {
            return fail(TBVH_ERR_WORKSPACE_TOO_SMALL, "%s: workspace of %zu bytes is smaller than the %zu needed", op,
                        ws_bytes, need);
        }
        TBVH_TRY(op, launch_grid_knn(a, node_aabbs, num_real_nodes, level, D, k, ws,
                                     static_cast<hipStream_t>(stream_ptr)));
        return ok();
    }
    TBVH_TRY(op, launch_knn_accel(a, D, k, false, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_knn_accel_grid_workspace_size(int64_t B, int64_t M, int64_t num_leaves, int D, int k, size_t* bytes) {
    const char* op = "tbvh_knn_accel_grid_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null output pointer", op);
    if (int r = check_dim(op, D)) return r;
    if (!supported_k(k)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: k must be 4, 8, 16 or 32, got %d", op, k);
    if (B < 1 || M < 0 || num_leaves < 1 || num_leaves > kMaxAccelCloud) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1, M >= 0 and num_leaves in [1, 2^28]", op);
    }
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    const int level = grid_level(num_leaves, D, k);
    *bytes = level > 0 ? grid_workspace_bytes(B, B * M, level, D) : 0;
    return ok();
}

int tbvh_knn_accel_grid(const void* accel, const float* node_aabbs, int64_t num_real_nodes, const float* queries,
                        const int64_t* order, int64_t B, int64_t M, int64_t num_leaves, int D, int k,
                        int64_t* out_indices, float* out_distances, void* ws, size_t ws_bytes, void* stream_ptr) {
    return knn_accel_batched("tbvh_knn_accel_grid", accel, queries, order, B, M, num_leaves, D, k, false,
                             out_indices, out_distances, stream_ptr, nullptr, 0, nullptr, node_aabbs,
                             num_real_nodes, ws ? ws : nullptr, ws_bytes);
}

int tbvh_knn_accel(const void* accel, const float* queries, const int64_t* order, int64_t B,
                   int64_t M, int64_t num_leaves, int D, int k, int64_t* out_indices,
                   float* out_distances, void* stream_ptr) {
    return knn_accel_batched("tbvh_knn_accel", accel, queries, order, B, M, num_leaves, D, k, false,
                             out_indices, out_distances, stream_ptr);
}

int tbvh_knn_accel_grid_spatial(const void* accel, const float* node_aabbs, int64_t num_real_nodes,
                                const float* queries, const int64_t* order, int64_t B, int64_t M, int64_t num_leaves,
                                int D, int k, int64_t* out_indices, float* out_distances, void* ws, size_t ws_bytes,
                                void* stream_ptr) {
    return knn_accel_batched("tbvh_knn_accel_grid_spatial", accel, queries, order, B, M, num_leaves, D, k, true,
                             out_indices, out_distances, stream_ptr, nullptr, 0, nullptr, node_aabbs, num_real_nodes,
                             ws, ws_bytes);
}

int tbvh_knn_accel_spatial(const void* accel, const float* queries, const int64_t* order, int64_t B,
                           int64_t M, int64_t num_leaves, int D, int k, int64_t* out_indices,
                           float* out_distances, void* stream_ptr) {
    return knn_accel_batched("tbvh_knn_accel_spatial", accel, queries, order, B, M, num_leaves, D, k,
                             true, out_indices, out_distances, stream_ptr);
}

static int knn_accel_ragged(const char* op, const void* accel, const int64_t* point_offsets,
                            int64_t total_points, const float* queries, const int64_t* query_offsets,
                            const int64_t* order, int64_t B, int64_t total_q, int D, int k,
                            int64_t* out_indices, float* out_distances, void* stream_ptr,
                            const float* source_points, int source_cols, float* out_positions) {
    if (int r = check_dim(op, D)) return r;
    if (!supported_k(k)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: k must be 4, 8, or 16 (32 is also supported), got %d", op, k);
    if (B < 1 || total_q < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and total_q >= 0", op);
    if (total_q > kMaxRows || total_points > kMaxRows || total_points < B) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: counts must fit in signed int32 (and total_points >= B)", op);
    }
    if (total_q == 0) return ok();
    if (!accel || !point_offsets || !queries || !query_offsets || !out_indices || !out_distances) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (!aligned(accel)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accel must be %zu-byte aligned", op, kAlign);
    KnnArgs a{};
    a.queries = queries;
    a.order = order;
    a.point_offsets = point_offsets;
    a.query_offsets = query_offsets;
    a.B = B;
    a.total_q = total_q;
    a.out_indices = out_indices;
    a.out_distances = out_distances;
    a.accel = accel;
    a.total_points = total_points;
    a.source_points = source_points;
    a.source_cols = source_cols;
    a.out_positions = out_positions;
    TBVH_TRY(op, launch_knn_accel(a, D, k, true, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_knn_accel_ragged(const void* accel, const int64_t* point_offsets, int64_t total_points,
                          const float* queries, const int64_t* query_offsets, const int64_t* order,
                          int64_t B, int64_t total_q, int D, int k, int64_t* out_indices,
                          float* out_distances, void* stream_ptr) {
    return knn_accel_ragged("tbvh_knn_accel_ragged", accel, point_offsets, total_points, queries,
                            query_offsets, order, B, total_q, D, k, out_indices, out_distances, stream_ptr,
                            nullptr, 0, nullptr);
}

static int check_positions(const char* op, const float* source_points, int source_cols, float* out_positions) {
    if (!source_points || !out_positions) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null source or positions pointer", op);
    if (source_cols < 1 || source_cols > 4096) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: source_cols must be in [1, 4096], got %d", op, source_cols);
    }
    return 0;
}

int tbvh_knn_accel_positions(const void* accel, const float* queries, const int64_t* order, int64_t B,
                             int64_t M, int64_t num_leaves, int D, int k, const float* source_points,
                             int source_cols, int64_t* out_indices, float* out_distances,
                             float* out_positions, void* stream_ptr) {
    const char* op = "tbvh_knn_accel_positions";
    if (int r = check_positions(op, source_points, source_cols, out_positions)) return r;
    return knn_accel_batched(op, accel, queries, order, B, M, num_leaves, D, k, false, out_indices,
                             out_distances, stream_ptr, source_points, source_cols, out_positions);
}

int tbvh_knn_accel_grid_positions(const void* accel, const float* node_aabbs, int64_t num_real_nodes,
                                  const float* queries, const int64_t* order, int64_t B, int64_t M,
                                  int64_t num_leaves, int D, int k, const float* source_points, int source_cols,
                                  int64_t* out_indices, float* out_distances, float* out_positions, void* ws,
                                  size_t ws_bytes, void* stream_ptr) {
    const char* op = "tbvh_knn_accel_grid_positions";
    if (int r = check_positions(op, source_points, source_cols, out_positions)) return r;
    return knn_accel_batched(op, accel, queries, order, B, M, num_leaves, D, k, false, out_indices, out_distances,
                             stream_ptr, source_points, source_cols, out_positions, node_aabbs, num_real_nodes,
                             ws, ws_bytes);
}

int tbvh_knn_accel_ragged_positions(const void* accel, const int64_t* point_offsets, int64_t total_points,
                                    const float* queries, const int64_t* query_offsets, const int64_t* order,
                                    int64_t B, int64_t total_q, int D, int k, const float* source_points,
                                    int source_cols, int64_t* out_indices, float* out_distances,
                                    float* out_positions, void* stream_ptr) {
    const char* op = "tbvh_knn_accel_ragged_positions";
    if (int r = check_positions(op, source_points, source_cols, out_positions)) return r;
    return knn_accel_ragged(op, accel, point_offsets, total_points, queries, query_offsets, order, B, total_q,
                            D, k, out_indices, out_distances, stream_ptr, source_points, source_cols,
                            out_positions);
}

// ---------------------------------------------------------------------------
// Routed k-NN (spatial output)
// ---------------------------------------------------------------------------
static int check_routed(const char* op, int64_t B, int64_t M, int64_t true_n, int64_t false_n, int64_t max_n,
                        int D, int k) {
    if (int r = check_dim(op, D)) return r;
    if (!supported_k(k)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: k must be 4, 8, or 16 (32 is also supported), got %d", op, k);
    if (B < 1 || M < 0) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 1 and M >= 0", op);
    if (true_n < 1 || true_n > max_n || false_n < 1 || false_n > max_n) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: leaf counts out of range", op);
    }
    if (true_n < k || false_n < k) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: both source counts must be >= k", op);
    if (M > 0 && B > kMaxRows / M) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total query count must fit in signed int32", op);
    if (B > kMaxRows / (true_n + false_n)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: total point count must fit in signed int32", op);
    }
    return TBVH_OK;
}

int tbvh_knn_routed_spatial(const float* true_node_aabbs, const int64_t* true_sorted_indices,
                            const float* false_node_aabbs, const int64_t* false_sorted_indices,
                            const float* queries, const uint8_t* routes, const int64_t* order, int64_t B,
                            int64_t M, int64_t true_num_leaves, int64_t true_num_real_nodes,
                            int64_t false_num_leaves, int64_t false_num_real_nodes, int D, int k,
                            int64_t* out_indices, float* out_distances, void* stream_ptr) {
    const char* op = "tbvh_knn_routed_spatial";
    if (int r = check_routed(op, B, M, true_num_leaves, false_num_leaves, kMaxCloud, D, k)) return r;
    if (true_num_real_nodes != tree::real_node_count(static_cast<int>(true_num_leaves)) ||
        false_num_real_nodes != tree::real_node_count(static_cast<int>(false_num_leaves))) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_real_nodes does not match num_leaves", op);
    }
    if (M == 0) return ok();
    if (!true_node_aabbs || !true_sorted_indices || !false_node_aabbs || !false_sorted_indices || !queries ||
        !routes || !order || !out_indices || !out_distances) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    KnnArgs a{};
    a.node_aabbs = true_node_aabbs;
    a.sorted_indices = true_sorted_indices;
    a.node_aabbs2 = false_node_aabbs;
    a.sorted_indices2 = false_sorted_indices;
    a.queries = queries;
    a.order = order;
    a.routes = routes;
    a.B = B;
    a.M = M;
    a.total_q = B * M;
    a.num_leaves = static_cast<int32_t>(true_num_leaves);
    a.num_real_nodes = static_cast<int32_t>(true_num_real_nodes);
    a.num_leaves2 = static_cast<int32_t>(false_num_leaves);
    a.num_real_nodes2 = static_cast<int32_t>(false_num_real_nodes);
    a.out_indices = out_indices;
    a.out_distances = out_distances;
    a.spatial_output = true;
    TBVH_TRY(op, launch_knn(a, D, k, false, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

// The routed accel traversal's arguments, checked (shared by the plain and
// the cell-block entry points).
static int routed_accel_args(const char* op, const void* true_accel, const void* false_accel,
                             const float* queries, const uint8_t* routes, const int64_t* order, int64_t B,
                             int64_t M, int64_t true_num_leaves, int64_t false_num_leaves, int D, int k,
                             int64_t* out_indices, float* out_distances, KnnArgs& a) {
    if (int r = check_routed(op, B, M, true_num_leaves, false_num_leaves, kMaxAccelCloud, D, k)) return r;
    if (M == 0) return ok();
    if (!true_accel || !false_accel || !queries || !routes || !order || !out_indices || !out_distances) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    if (!aligned(true_accel) || !aligned(false_accel)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: accels must be %zu-byte aligned", op, kAlign);
    }
    a = KnnArgs{};
    a.queries = queries;
    a.order = order;
    a.routes = routes;
    a.B = B;
    a.M = M;
    a.total_q = B * M;
    a.num_leaves = static_cast<int32_t>(true_num_leaves);
    a.num_leaves2 = static_cast<int32_t>(false_num_leaves);
    a.accel = true_accel;
    a.accel2 = false_accel;
    a.total_points = B * true_num_leaves;
    a.out_indices = out_indices;
    a.out_distances = out_distances;
    a.spatial_output = true;
    return TBVH_OK;
}

int tbvh_knn_accel_routed_spatial(const void* true_accel, const void* false_accel, const float* queries,
                                  const uint8_t* routes, const int64_t* order, int64_t B, int64_t M,
                                  int64_t true_num_leaves, int64_t false_num_leaves, int D, int k,
                                  int64_t* out_indices, float* out_distances, void* stream_ptr) {
    const char* op = "tbvh_knn_accel_routed_spatial";
    KnnArgs a{};
    if (int r = routed_accel_args(op, true_accel, false_accel, queries, routes, order, B, M, true_num_leaves,
                                  false_num_leaves, D, k, out_indices, out_distances, a)) {
        return r;
    }
    if (M == 0) return ok();
    TBVH_TRY(op, launch_knn_accel(a, D, k, false, static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

int tbvh_knn_accel_routed_grid_workspace_size(int64_t B, int64_t M, int64_t true_num_leaves,
                                              int64_t false_num_leaves, int D, int k, size_t* bytes) {
    const char* op = "tbvh_knn_accel_routed_grid_workspace_size";
    if (!bytes) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null output pointer", op);
    if (int r = check_routed(op, B, M, true_num_leaves, false_num_leaves, kMaxAccelCloud, D, k)) return r;
    const int level = grid_level(true_num_leaves, D, k);
    const int level2 = grid_level(false_num_leaves, D, k);
    *bytes = level > 0 && level2 > 0 ? grid_workspace_bytes(B, B * M, level, D, level2) : 0;
    return ok();
}

int tbvh_knn_accel_routed_grid_spatial(const void* true_accel, const float* true_node_aabbs,
                                       int64_t true_num_real_nodes, const void* false_accel,
                                       const float* false_node_aabbs, int64_t false_num_real_nodes,
                                       const float* queries, const uint8_t* routes, const int64_t* order,
                                       int64_t B, int64_t M, int64_t true_num_leaves, int64_t false_num_leaves,
                                       int D, int k, int64_t* out_indices, float* out_distances, void* ws,
                                       size_t ws_bytes, void* stream_ptr) {
    const char* op = "tbvh_knn_accel_routed_grid_spatial";
    KnnArgs a{};
    if (int r = routed_accel_args(op, true_accel, false_accel, queries, routes, order, B, M, true_num_leaves,
                                  false_num_leaves, D, k, out_indices, out_distances, a)) {
        return r;
    }
    if (M == 0) return ok();
    const hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
    const int level = ws ? grid_level(true_num_leaves, D, k) : 0;
    const int level2 = ws ? grid_level(false_num_leaves, D, k) : 0;
    if (level > 0 && level2 > 0) {
        if (!true_node_aabbs || !false_node_aabbs) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null node_aabbs", op);
        if (true_num_real_nodes != tree::real_node_count(static_cast<int>(true_num_leaves)) ||
            false_num_real_nodes != tree::real_node_count(static_cast<int>(false_num_leaves))) {
            return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: num_real_nodes does not match num_leaves", op);
        }
        if (!aligned(ws)) return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: workspace must be %zu-byte aligned", op, kAlign);
        const size_t need = grid_workspace_bytes(B, B * M, level, D, level2);
        if (ws_bytes < need) {
            return fail(TBVH_ERR_WORKSPACE_TOO_SMALL, "%s: workspace of %zu bytes is smaller than the %zu needed", op,
                        ws_bytes, need);
        }
        TBVH_TRY(op, launch_grid_knn(a, true_node_aabbs, true_num_real_nodes, level, D, k, ws, stream,
                                     false_node_aabbs, false_num_real_nodes, level2));
        return ok();
    }
    TBVH_TRY(op, launch_knn_accel(a, D, k, false, stream));
    return ok();
}

int tbvh_interpolate_neighbors(const float* values, const int64_t* indices, const float* weights,
                               const uint8_t* exact, int64_t B, int64_t N, int64_t H, int64_t C, int k,
                               float* out, void* stream_ptr) {
    const char* op = "tbvh_interpolate_neighbors";
    if (B < 0 || N < 0 || H < 1 || C < 1 || k < 1) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: need B >= 0, N >= 0, H >= 1, C >= 1 and k >= 1", op);
    }
    // Checked products: sizes come from the caller.
    int64_t rows = 0, items = 0;
    if (__builtin_mul_overflow(B, N, &rows) || __builtin_mul_overflow(rows, H, &rows) ||
        __builtin_mul_overflow(rows, C, &items) || items > (int64_t{1} << 40)) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: B * N * H * C exceeds 2^40", op);
    }
    if (rows == 0) return ok();
    if (!values || !indices || !weights || !exact || !out) {
        return fail(TBVH_ERR_INVALID_ARGUMENT, "%s: null input or output pointer", op);
    }
    TBVH_TRY(op, launch_interpolate(values, indices, weights, exact, rows, N, H, C, k, out,
                                    static_cast<hipStream_t>(stream_ptr)));
    return ok();
}

}  // extern "C"
