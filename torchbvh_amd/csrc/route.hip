// Routed query ordering: each query of cloud b carries a route (true/false)
// naming one of two BVHs; the order is the stable order of the composite key
// (route above the Morton code of the query against that route's bounds),
// per cloud (reference: `morton_sort_routed_queries_batched`,
// torchbvh/csrc/morton_sort.cu:82-120, 288-329).
//
// The composite has 31 (3-D) or 33 (2-D) bits, so it is not sorted as one
// key.  Instead: (1) a one-pass stable sort on the route digit partitions
// each cloud into its false queries then its true queries, in query order;
// (2) the partitioned queries are gathered, each group becoming a segment
// with its route's bounds; (3) the ordinary segmented Morton sort orders
// every segment; (4) segment-local positions are mapped back to query
// indices.  Stable partition followed by a stable sort within each group is
// exactly the stable sort of (route, code).
#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

// Route digits (0/1) of every query and each tile's digit counts (the
// sort's first-pass input: [digit][tile], zero beyond digit 1 and for
// surplus tiles).
__global__ __launch_bounds__(kBlock) void route_keys_kernel(const uint8_t* __restrict__ routes,
                                                            const Segment* __restrict__ segs, int S,
                                                            uint32_t* __restrict__ keys,
                                                            uint32_t* __restrict__ tile_hist,
                                                            int64_t tstride) {
    static_assert(kBlock == kRadix, "one thread per digit");
    __shared__ int s_seg;
    __shared__ uint32_t s_ones;
    const int64_t t = blockIdx.x;
    if (threadIdx.x == 0) s_ones = 0u;
    const int s = block_find_segment([&](int i) { return static_cast<int64_t>(segs[i].tile_first); },
                                     S, t, &s_seg);
    const Segment g = segs[s];
    const int lt = static_cast<int>(t - g.tile_first);
    int count = 0;
    if (lt < g.tiles) {
        const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
        count = min(kSortTile, g.n - lt * kSortTile);
        uint32_t ones = 0;
        for (int j = threadIdx.x; j < count; j += kBlock) {
            const uint32_t r = routes[row0 + j] != 0 ? 1u : 0u;
            keys[row0 + j] = r;
            ones += r;
        }
        ones = wave_sum(ones);
        if (lane_id() == 0) atomicAdd(&s_ones, ones);
    }
    __syncthreads();
    const uint32_t c1 = s_ones;
    const uint32_t c = threadIdx.x == 0 ? static_cast<uint32_t>(count) - c1 : (threadIdx.x == 1 ? c1 : 0u);
    tile_hist[threadIdx.x * tstride + t] = c;
}

// Queries in partitioned order, the 2B group segments and their bounds.
template <int D>
__global__ __launch_bounds__(kBlock) void route_gather_kernel(
    const float* __restrict__ queries, const int64_t* __restrict__ part, const Segment* __restrict__ segs,
    const uint32_t* __restrict__ tile_scan, int64_t B, int64_t M, const float* __restrict__ true_min,
    const float* __restrict__ true_max,
    const float* __restrict__ false_min, const float* __restrict__ false_max, float* __restrict__ gathered,
    int64_t* __restrict__ group_offsets, float* __restrict__ group_min, float* __restrict__ group_max) {
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= B * M) return;
    const int64_t b = j / M;
    const int64_t m = min(max(part[j], int64_t(0)), M - 1);
#pragma unroll
    for (int d = 0; d < D; ++d) gathered[j * D + d] = queries[(b * M + m) * D + d];
    if (j - b * M == 0) {
        // False queries of cloud b: digit 0's count over the cloud's tiles
        // (row 0 of the route sort's tile scan).
        const Segment g = segs[b];
        const int64_t c0 = tile_scan[g.tile_first + g.tiles] - tile_scan[g.tile_first];
        group_offsets[2 * b] = b * M;
        group_offsets[2 * b + 1] = b * M + c0;
        if (b == B - 1) group_offsets[2 * B] = B * M;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            group_min[(2 * b) * D + d] = false_min[b * D + d];
            group_max[(2 * b) * D + d] = false_max[b * D + d];
            group_min[(2 * b + 1) * D + d] = true_min[b * D + d];
            group_max[(2 * b + 1) * D + d] = true_max[b * D + d];
        }
    }
}

// order[b, i] = query index of position i: the group-local sorted position
// mapped through the partition.
__global__ __launch_bounds__(kBlock) void route_finish_kernel(const int64_t* __restrict__ part,
                                                              const int64_t* __restrict__ sorted_local,
                                                              const int64_t* __restrict__ group_offsets,
                                                              int64_t B, int64_t M,
                                                              int64_t* __restrict__ order) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= B * M) return;
    const int64_t b = i / M;
    const int64_t c0 = group_offsets[2 * b + 1] - b * M;
    const int64_t group_start = (i - b * M) < c0 ? 0 : c0;
    const int64_t local = min(max(sorted_local[i], int64_t(0)), M - 1);
    const int64_t at = min(group_start + local, M - 1);
    order[i] = part[b * M + at];
}

inline unsigned grid_for(int64_t items) { return static_cast<unsigned>((items + kBlock - 1) / kBlock); }

}  // namespace

hipError_t launch_route_keys(const uint8_t* routes, const Segment* segs, int64_t S, int64_t tiles,
                             uint32_t* keys, uint32_t* tile_hist, int64_t tstride, hipStream_t stream) {
    route_keys_kernel<<<static_cast<unsigned>(tiles), kBlock, 0, stream>>>(routes, segs, static_cast<int>(S),
                                                                           keys, tile_hist, tstride);
    return hipGetLastError();
}

hipError_t launch_route_gather(const float* queries, const int64_t* part, const Segment* segs,
                               const uint32_t* tile_scan, int64_t B,
                               int64_t M, int D, const float* true_min, const float* true_max,
                               const float* false_min, const float* false_max, float* gathered,
                               int64_t* group_offsets, float* group_min, float* group_max,
                               hipStream_t stream) {
    if (D == 3) {
        route_gather_kernel<3><<<grid_for(B * M), kBlock, 0, stream>>>(
            queries, part, segs, tile_scan, B, M, true_min, true_max, false_min, false_max, gathered,
            group_offsets, group_min, group_max);
    } else {
        route_gather_kernel<2><<<grid_for(B * M), kBlock, 0, stream>>>(
            queries, part, segs, tile_scan, B, M, true_min, true_max, false_min, false_max, gathered,
            group_offsets, group_min, group_max);
    }
    return hipGetLastError();
}

hipError_t launch_route_finish(const int64_t* part, const int64_t* sorted_local, const int64_t* group_offsets,
                               int64_t B, int64_t M, int64_t* order, hipStream_t stream) {
    route_finish_kernel<<<grid_for(B * M), kBlock, 0, stream>>>(part, sorted_local, group_offsets, B, M,
                                                                 order);
    return hipGetLastError();
}

}  // namespace tbvh
