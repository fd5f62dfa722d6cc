// Neighbour-value accumulation of interpolate_displaced.
//
// The reference loops over the k neighbour ranks in Python, each step a
// gather of the neighbours' rows and two broadcast multiply-adds over the
// whole (B, N, H, Ch) tensor, and finally, after asking the host whether any
// exact hit exists, swaps in the plain mean of the exact hits
// (torchbvh/_multihead.py:123-144).  Here one thread owns V channels of one
// query row and walks the ranks in the same order with the same two
// roundings per step (product, then sum; the library is built with
// -ffp-contract=off), so both sums are bit-identical, the exact-hit count
// is a sum of ones and the mean is one correctly rounded division, as in
// the reference.  No gathered rows are materialised and no host
// synchronisation decides whether any exact hit exists.
#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

constexpr int64_t kMaxGrid = int64_t{1} << 20;  // work-groups per launch

template <int V>
struct Vec;
template <>
struct Vec<1> {
    using T = float;
};
template <>
struct Vec<4> {
    using T = float4;
};

template <int V>
__device__ __forceinline__ float lane(const typename Vec<V>::T& v, int i) {
    if constexpr (V == 1) {
        return v;
    } else {
        return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
    }
}

template <int V>
__device__ __forceinline__ void interpolate_item(const float* __restrict__ values,
                                                 const int64_t* __restrict__ indices,
                                                 const float* __restrict__ weights,
                                                 const uint8_t* __restrict__ exact, int64_t t, int64_t groups,
                                                 int64_t N, int64_t H, int64_t C, int K, float* __restrict__ out) {
    using T = typename Vec<V>::T;
    const int64_t r = t / groups;              // query row (b, n, h)
    const int64_t c = (t - r * groups) * V;    // first channel
    const int64_t h = r % H;
    const int64_t b = r / (N * H);
    float acc[V], ex[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = ex[i] = 0.0f;
    float hits = 0.0f;
    for (int j = 0; j < K; ++j) {
        const int64_t idx = indices[r * K + j];
        const float w = weights[r * K + j];
        const float e = exact[r * K + j] ? 1.0f : 0.0f;
        hits = hits + e;
        T v{};
        if (idx >= 0 && idx < N) v = *reinterpret_cast<const T*>(values + ((b * N + idx) * H + h) * C + c);
#pragma unroll
        for (int i = 0; i < V; ++i) {
            const float x = lane<V>(v, i);
            acc[i] = acc[i] + x * w;
            ex[i] = ex[i] + x * e;
        }
    }
    T res;
    float* o = reinterpret_cast<float*>(&res);
#pragma unroll
    for (int i = 0; i < V; ++i) o[i] = hits > 0.0f ? ex[i] / hits : acc[i];
    *reinterpret_cast<T*>(out + r * C + c) = res;
}

// Grid-stride over (row, channel group) items: the grid is capped, since a
// launch holds fewer than 2^32 work-items.
template <int V>
__global__ __launch_bounds__(kBlock) void interpolate_kernel(const float* __restrict__ values,
                                                             const int64_t* __restrict__ indices,
                                                             const float* __restrict__ weights,
                                                             const uint8_t* __restrict__ exact, int64_t rows,
                                                             int64_t N, int64_t H, int64_t C, int K,
                                                             float* __restrict__ out) {
    const int64_t groups = C / V;  // V-channel groups per row
    const int64_t items = rows * groups;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; t < items; t += stride) {
        interpolate_item<V>(values, indices, weights, exact, t, groups, N, H, C, K, out);
    }
}

}  // namespace

hipError_t launch_interpolate(const float* values, const int64_t* indices, const float* weights,
                              const uint8_t* exact, int64_t rows, int64_t N, int64_t H, int64_t C, int K,
                              float* out, hipStream_t stream) {
    const bool vec = C % 4 == 0 && reinterpret_cast<uintptr_t>(values) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(out) % 16 == 0;
    const int64_t items = rows * (vec ? C / 4 : C);
    if (items == 0) return hipSuccess;
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>((items + kBlock - 1) / kBlock, kMaxGrid));
    if (vec) {
        interpolate_kernel<4><<<grid, kBlock, 0, stream>>>(values, indices, weights, exact, rows, N, H, C, K, out);
    } else {
        interpolate_kernel<1><<<grid, kBlock, 0, stream>>>(values, indices, weights, exact, rows, N, H, C, K, out);
    }
    return hipGetLastError();
}

}  // namespace tbvh
