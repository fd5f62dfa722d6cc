// Small clouds in one work-group each: bounds, keys and the whole stable
// key/value sort in LDS, one launch.
//
// For clouds of up to kSmallCloud rows this replaces the bounds, Morton and
// eleven sort launches of the general sequence (tile counts, scans and
// scatters of four 8-bit passes, sort.hip), whose fixed costs set the time
// of a small build: at 10,000 points those thirteen launches take ~65 us of
// kernel time for 40 kB of keys.  Everything stays in one work-group of
// kSmallThreads threads, and every pass is the same stable counting sort as
// the general scatter (wave64 ballot ranking, per-wave digit counters, LDS
// staging in digit order), so the order is identical: ties in the key keep
// ascending original index (the CUB contract the sort replaces,
// bvh_build.cu:580-594), and the bounds are the same fminf/fmaxf reductions
// from the same seeds (bvh_build.cu:453-494).
#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

constexpr int kSmallThreads = 1024;
constexpr int kSmallWaves = kSmallThreads / kWave;

// One cloud per work-group (segment blockIdx.x).  The cloud's rows are dealt
// to all the waves in contiguous ranges of `per_wave` rows (a multiple of
// 64, the fewest that cover it): row j = w * per_wave + i * 64 + l is item i
// of lane l of wave w, so ranking within a wave is ranking in row order, and
// a wave's serial ranking chain is per_wave / 64 = ceil(n / 1024) items long
// whatever kItems is (one item per 1,024 rows: 10 at 10,000 rows, not 16).
// With `bounds`, the cloud's box from (seed_lo, seed_hi) is stored into
// scene_min/max and keys the rows against it; otherwise scene_min/max are
// read.  Passes sort 8-bit digits from first_bit up; the cloud-local order
// goes to `order` (int64) and, if given, the sorted keys to `sorted_keys`.
template <int D, int kItems, bool kHilbert>
__global__ __launch_bounds__(kSmallThreads) void small_sort_kernel(
    const float* __restrict__ rows, const Segment* segs, int S, UniformPlan plan, float* __restrict__ scene_min,
    float* __restrict__ scene_max, bool bounds, float seed_lo, float seed_hi, int first_bit, int passes,
    int64_t* __restrict__ order, uint32_t* __restrict__ sorted_keys) {
    constexpr int kCap = kItems * kSmallThreads;
    __shared__ uint32_t s_keys[kCap];
    __shared__ uint32_t s_vals[kCap];
    __shared__ uint32_t s_cnt[kSmallWaves][kRadix];
    __shared__ uint32_t s_start[kRadix];
    __shared__ uint32_t s_scan[kSmallWaves];
    __shared__ float s_red[kSmallWaves][2 * D];
    __shared__ float s_box[2 * D];
    const int s = blockIdx.x;
    if (plan.table) store_uniform_table(plan.table, S, plan.n, plan.tree);
    const Segment g = plan.n > 0 ? uniform_segment(s, plan.n, plan.tree) : segs[s];
    const int n = g.n;
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const int per_wave = (n + kSmallThreads - 1) / kSmallThreads * kWave;
    const int base = wave * per_wave + lane;
    // Item i of this lane is a row of the cloud (the first test is wave-uniform).
    auto valid = [&](int i) { return i * kWave < per_wave && base + i * kWave < n; };

    // The rows are read twice (bounds, then keys; the second read hits in
    // cache), kChunk rows per thread at a time: the loads of a chunk issue
    // together (rows past the cloud read its last row and are masked), so
    // the work-group waits kItems / kChunk round trips per sweep instead of
    // kItems, and no thread holds all its rows (which spills at 16).
    constexpr int kChunk = kItems % 8 == 0 ? 8 : 4;
    static_assert(kItems % kChunk == 0, "whole chunks of rows");
    const PointRow<D>* src = reinterpret_cast<const PointRow<D>*>(rows + g.start * D);
    float lo[D], hi[D];
    if (bounds) {
#pragma unroll
        for (int d = 0; d < D; ++d) { lo[d] = seed_lo; hi[d] = seed_hi; }
#pragma unroll
        for (int c = 0; c < kItems; c += kChunk) {
            PointRow<D> r[kChunk];
#pragma unroll
            for (int u = 0; u < kChunk; ++u) r[u] = src[min(base + (c + u) * kWave, n - 1)];
#pragma unroll
            for (int u = 0; u < kChunk; ++u) {
                if (valid(c + u)) {
#pragma unroll
                    for (int d = 0; d < D; ++d) {
                        lo[d] = fminf(lo[d], r[u].v[d]);
                        hi[d] = fmaxf(hi[d], r[u].v[d]);
                    }
                }
            }
        }
        block_box<D, kSmallThreads>(lo, hi, s_red, s_box);
        __syncthreads();
#pragma unroll
        for (int d = 0; d < D; ++d) { lo[d] = s_box[d]; hi[d] = s_box[D + d]; }
        if (threadIdx.x < D) {
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
    uint32_t key[kItems], val[kItems];
#pragma unroll
    for (int c = 0; c < kItems; c += kChunk) {
        PointRow<D> r[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) r[u] = src[min(base + (c + u) * kWave, n - 1)];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const int i = c + u;
            const int j = base + i * kWave;
            key[i] = valid(i) ? (kHilbert ? hilbert::schedule_key<D>(r[u].v, lo, hi) : morton::encode<D>(r[u].v, lo, hi))
                              : 0xffffffffu;
            val[i] = static_cast<uint32_t>(j);
        }
    }

    const uint64_t below = (1ull << lane) - 1ull;
    for (int p = 0; p < passes; ++p) {
        const int shift = first_bit + p * kRadixBits;
        for (int i = threadIdx.x; i < kSmallWaves * kRadix; i += kSmallThreads) (&s_cnt[0][0])[i] = 0u;
        __syncthreads();
        // Stable rank of each key among this wave's keys of its digit.
        uint32_t rank[kItems];
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            rank[i] = 0;
            if (i * kWave >= per_wave) continue;  // the wave's rows end before this item
            const bool ok = base + i * kWave < n;
            const uint32_t digit = (key[i] >> shift) & (kRadix - 1);
            const uint64_t peers = match_digit(digit, ok);
            const uint32_t before = static_cast<uint32_t>(__popcll(peers & below));
            const uint32_t prior = ok ? s_cnt[wave][digit] : 0u;
            __builtin_amdgcn_wave_barrier();
            if (ok && before == 0) s_cnt[wave][digit] = prior + static_cast<uint32_t>(__popcll(peers));
            __builtin_amdgcn_wave_barrier();
            rank[i] = prior + before;
        }
        __syncthreads();
        // Thread d < kRadix: the digit's counts in earlier waves, and the
        // cloud's keys of smaller digits.
        const int d = threadIdx.x;
        uint32_t count = 0;
        if (d < kRadix) {
#pragma unroll
            for (int w = 0; w < kSmallWaves; ++w) {
                const uint32_t c = s_cnt[w][d];
                s_cnt[w][d] = count;
                count += c;
            }
        }
        const uint32_t start = block_exclusive_sum<kSmallThreads>(count, s_scan);
        if (d < kRadix) s_start[d] = start;
        __syncthreads();
        // A key's place: smaller digits, then its digit in earlier waves,
        // then earlier in its own wave: a bijection onto [0, n).
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            if (valid(i)) {
                const uint32_t digit = (key[i] >> shift) & (kRadix - 1);
                const uint32_t at = s_start[digit] + s_cnt[wave][digit] + rank[i];
                s_keys[at] = key[i];
                s_vals[at] = val[i];
            }
        }
        __syncthreads();
        if (p + 1 < passes) {
#pragma unroll
            for (int i = 0; i < kItems; ++i) {
                if (valid(i)) {
                    key[i] = s_keys[base + i * kWave];
                    val[i] = s_vals[base + i * kWave];
                }
            }
        }
    }
    for (int j = threadIdx.x; j < n; j += kSmallThreads) {
        order[g.start + j] = static_cast<int64_t>(s_vals[j]);
        if (sorted_keys) sorted_keys[g.start + j] = s_keys[j];
    }
}

template <int D, int kItems>
void launch_items(const float* rows, const Segment* segs, int64_t S, UniformPlan plan, float* scene_min,
                  float* scene_max, bool bounds, float seed_lo, float seed_hi, SortBits bits, int64_t* order,
                  uint32_t* sorted_keys, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(S);
    if (bits.hilbert) {
        small_sort_kernel<D, kItems, true><<<grid, kSmallThreads, 0, stream>>>(
            rows, segs, static_cast<int>(S), plan, scene_min, scene_max, bounds, seed_lo, seed_hi, bits.first_bit,
            bits.passes(), order, sorted_keys);
    } else {
        small_sort_kernel<D, kItems, false><<<grid, kSmallThreads, 0, stream>>>(
            rows, segs, static_cast<int>(S), plan, scene_min, scene_max, bounds, seed_lo, seed_hi, bits.first_bit,
            bits.passes(), order, sorted_keys);
    }
}

template <int D>
void launch_d(const float* rows, const Segment* segs, int64_t S, UniformPlan plan, int64_t max_n, float* scene_min,
              float* scene_max, bool bounds, float seed_lo, float seed_hi, SortBits bits, int64_t* order,
              uint32_t* sorted_keys, hipStream_t stream) {
    // Up to 4 keys per thread (48 kB of LDS) to 4,096 rows, else up to 12
    // (112 kB).  At 16 keys per thread (16,384 rows) this kernel measured
    // slower than the general sequence (full build 130.6 against 121.5 us at
    // 16,384 points), at 10,000 points faster (107.4 against 120.5 us).
    if (max_n <= 4 * kSmallThreads) {
        launch_items<D, 4>(rows, segs, S, plan, scene_min, scene_max, bounds, seed_lo, seed_hi, bits, order,
                           sorted_keys, stream);
    } else {
        launch_items<D, kSmallCloud / kSmallThreads>(rows, segs, S, plan, scene_min, scene_max, bounds, seed_lo,
                                                     seed_hi, bits, order, sorted_keys, stream);
    }
}

}  // namespace

hipError_t launch_small_sort(const float* rows, int D, const Segment* segs, int64_t S, UniformPlan plan,
                             int64_t max_n, float* scene_min, float* scene_max, bool bounds, float seed_lo,
                             float seed_hi, SortBits bits, int64_t* order, uint32_t* sorted_keys,
                             hipStream_t stream) {
    if (max_n > kSmallCloud || S < 1) return hipErrorInvalidValue;
    if (D == 3) {
        launch_d<3>(rows, segs, S, plan, max_n, scene_min, scene_max, bounds, seed_lo, seed_hi, bits, order,
                    sorted_keys, stream);
    } else {
        launch_d<2>(rows, segs, S, plan, max_n, scene_min, scene_max, bounds, seed_lo, seed_hi, bits, order,
                    sorted_keys, stream);
    }
    return hipGetLastError();
}

}  // namespace tbvh
