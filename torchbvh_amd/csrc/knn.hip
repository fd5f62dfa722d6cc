// Exact k-NN by branch-and-bound over a BVH of one cloud.
//
// Follows the reference traversal (torchbvh/csrc/knn_query.cu:47-154): one
// query per lane, launched in Morton order when an order is given; at an
// internal node both real children's box distances are evaluated, the far
// child is deferred on a stack with its distance cached if it can still hold
// a candidate, and the near child is entered; nodes are visited while their
// box distance is <= the current k-th distance.  The same traversal runs over
// two node sources: the reference's implicit tree (node_aabbs + sorted
// indices) and the acceleration structure built beside it (accel.hip).
//
// The candidate list is where this kernel deliberately differs: entries are
// 64-bit keys (float bits of the squared distance << 32 | point index) kept
// in ascending order in registers.  Squared distances are >= 0, so their bit
// patterns order like the floats and one unsigned compare orders candidates
// lexicographically by (distance, index).  The result is therefore the k
// smallest (distance, index) pairs, independent of traversal order: exact
// ties resolve to the lower point index.  Empty slots hold (FLT_MAX, -1),
// the reference's initial values (knn_query.cu:13, :83-85).
//
// Distances: delta_d = max(lo - q, max(0, q - hi)) per axis (geometry.cuh:3-18)
// accumulated as fma(d2, d2, fma(d1, d1, d0 * d0)), the contraction the
// reference's `dist += delta * delta` loop compiles to.  On a leaf's
// degenerate box this is the exact point distance with delta = |q - p|.
#include <float.h>

#include <algorithm>
#include <cmath>

#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

constexpr float kFar = FLT_MAX;

template <int D>
__device__ __forceinline__ float box_distance(const float* q, const float* box) {
    float s = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const float delta = fmaxf(box[d] - q[d], fmaxf(0.0f, q[d] - box[D + d]));
        s = d == 0 ? delta * delta : __builtin_fmaf(delta, delta, s);
    }
    return s;
}

__device__ __forceinline__ uint64_t candidate_key(float dist, uint32_t idx) {
    return (static_cast<uint64_t>(__float_as_uint(dist)) << 32) | idx;
}

// Minimum / maximum of two candidate keys by f64 min / max.  A key read as
// an IEEE double is never negative and never NaN: its sign bit is the sign
// of a distance >= 0, and an all-ones exponent field would need a float
// distance with an all-ones exponent (inf/NaN), which is never inserted
// (the largest key holds FLT_MAX).  Such doubles order exactly like the
// 64-bit unsigned keys, and with f64 denormals kept (the default mode;
// distance-0 keys read as denormals) v_min_f64 / v_max_f64 return one
// operand bit for bit.  Written as instructions: the compiler's fmin/fmax
// would first canonicalise each operand, one more instruction per slot.
__device__ __forceinline__ uint64_t key_min(uint64_t a, uint64_t b) {
    double r;
    asm("v_min_f64 %0, %1, %2" : "=v"(r) : "v"(__longlong_as_double(a)), "v"(__longlong_as_double(b)));
    return static_cast<uint64_t>(__double_as_longlong(r));
}
__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) {
    double r;
    asm("v_max_f64 %0, %1, %2" : "=v"(r) : "v"(__longlong_as_double(a)), "v"(__longlong_as_double(b)));
    return static_cast<uint64_t>(__double_as_longlong(r));
}

// Insert `key` into the ascending list `best`, dropping the largest entry:
// slot i becomes min(best[i], max(best[i - 1], key)), which is best[i]
// below the insertion point, key at it and best[i - 1] above it.  Two
// independent instructions per slot (a compare-and-select chain needs a
// compare and four selects, serialised through the compare mask); measured
// on MI355X: traversal -7% at k = 16 (cfg2), -20% at k = 32 (cfg5).
template <int K>
__device__ __forceinline__ void insert_sorted(uint64_t (&best)[K], uint64_t key) {
#pragma unroll
    for (int i = K - 1; i > 0; --i) best[i] = key_min(best[i], key_max(best[i - 1], key));
    best[0] = key_min(best[0], key);
}

// The key of an empty slot, (FLT_MAX, -1): also what a candidate that may
// not enter the list (distance FLT_MAX, inf or NaN) becomes before a merge.
constexpr uint64_t kEmptyKey = (static_cast<uint64_t>(0x7f7fffffu) << 32) | 0xffffffffu;

__device__ __forceinline__ void key_exchange(uint64_t& lo, uint64_t& hi) {
    const uint64_t a = lo, b = hi;
    lo = key_min(a, b);
    hi = key_max(a, b);
}

// Ascending sort of a bucket's candidate keys by a fixed network: the
// optimal 12-comparator network for 6 inputs, Batcher's 19-comparator
// odd-even merge sort for 8 (Knuth, TAOCP vol. 3, 5.3.4).
// Sorts c[O .. O + B).
template <int B, int O = 0, int N>
__device__ __forceinline__ void sort_candidates(uint64_t (&c)[N]) {
    static_assert(B == 6 || B == 8, "bucket sizes are 6 (3-D) and 8 (2-D)");
    static_assert(O + B <= N, "range inside the array");
    if constexpr (B == 6) {
        constexpr int net[12][2] = {{0, 5}, {1, 3}, {2, 4}, {1, 2}, {3, 4}, {0, 3},
                                    {2, 5}, {0, 1}, {2, 3}, {4, 5}, {1, 2}, {3, 4}};
#pragma unroll
        for (int s = 0; s < 12; ++s) key_exchange(c[O + net[s][0]], c[O + net[s][1]]);
    } else {
        constexpr int net[19][2] = {{0, 2}, {1, 3}, {4, 6}, {5, 7}, {0, 4}, {1, 5}, {2, 6},
                                    {3, 7}, {0, 1}, {2, 3}, {4, 5}, {6, 7}, {2, 4}, {3, 5},
                                    {1, 4}, {3, 6}, {1, 2}, {3, 4}, {5, 6}};
#pragma unroll
        for (int s = 0; s < 19; ++s) key_exchange(c[O + net[s][0]], c[O + net[s][1]]);
    }
}

// Merge a bucket's candidates into the ascending list, keeping the K
// smallest keys: with the candidates sorted ascending, slot K - m + i takes
// min(best[K - m + i], c[m - 1 - i]) (a bitonic half-cleaner of the list
// against the reversed candidates), which leaves the K smallest keys of both
// as a bitonic sequence, and log2(K) rounds of compare-exchanges sort it
// (Batcher's bitonic merge).  The same K keys as inserting the candidates
// one by one, for (K/2)·log2(K) + m + the sort's comparators, with every
// lane of the wave busy: one insertion per accepted candidate ran once per
// candidate slot for the whole wave whenever any lane accepted that slot.
//
// A compare-exchange of two slots that both still hold the list's own
// entries (untouched by the half-cleaner and by every earlier exchange) is a
// no-op, since the list is sorted; MergePlan marks the others, so the merge
// runs 30 of 32 exchanges at K = 16 and 66 of 80 at K = 32 (6 candidates).
template <int K, int M>
struct MergePlan {
    static constexpr int kStages = K >= 32 ? 5 : K >= 16 ? 4 : K >= 8 ? 3 : K >= 4 ? 2 : 1;
    uint64_t needed[kStages] = {};  // stage s (stride K >> (s + 1)): bit i = exchange (i, i + stride) runs
    constexpr MergePlan() {
        uint64_t touched = ((uint64_t(1) << M) - 1) << (K - M);
        for (int s = 0, h = K / 2; h >= 1; ++s, h /= 2) {
            uint64_t next = touched;
            for (int i = 0; i < K; ++i) {
                if ((i & h) == 0 && (((touched >> i) | (touched >> (i + h))) & 1)) {
                    needed[s] |= uint64_t(1) << i;
                    next |= (uint64_t(1) << i) | (uint64_t(1) << (i + h));
                }
            }
            touched = next;
        }
    }
};

template <int K, int B, int kBarrierFromK = 32>
__device__ __forceinline__ void merge_candidates(uint64_t (&best)[K], uint64_t (&c)[B]) {
    sort_candidates<B>(c);
    constexpr int m = K < B ? K : B;
    constexpr MergePlan<K, m> plan{};
#pragma unroll
    for (int i = 0; i < m; ++i) best[K - m + i] = key_min(best[K - m + i], c[m - 1 - i]);
#pragma unroll
    for (int s = 0; s < MergePlan<K, m>::kStages; ++s) {
        const int h = K >> (s + 1);
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if ((i & h) == 0 && ((plan.needed[s] >> i) & 1)) key_exchange(best[i], best[i + h]);
        }
        // At K = 32 the scheduler would otherwise start the next stage's
        // exchanges before this one's maxima, holding up to 32 more VGPRs
        // (the cell-block search asks for this from K = 16).
        if constexpr (K >= kBarrierFromK) __builtin_amdgcn_sched_barrier(0);
    }
}

// Writes one result row: the K (index, distance) pairs and, when asked,
// the neighbours' source rows.  `pstart` is the cloud's first point row,
// `index_offset` what the routed traversal adds to false-route indices.
template <int C>
struct SourceRow {
    float v[C];
};

template <int K, int D = 0, bool kWideDist = false>
__device__ __forceinline__ void write_results(const KnnArgs& a, int64_t out_row, const uint64_t (&best)[K],
                                              int64_t index_offset, int64_t pstart) {
    int64_t* oi = a.out_indices + out_row * K;
    float* od = a.out_distances + out_row * K;
    // With kWideDist, the distance row as 16-byte stores where the output
    // allows (a wave-uniform test): each store of a wave writes 64 rows, so
    // four instead of sixteen at K = 16.  Measured at cfg2: the cell-block
    // second pass -2 us with them, the first pass +10 us (its registers
    // 87 -> 96, the same occupancy), so only the second pass asks.
    if (kWideDist && (reinterpret_cast<uintptr_t>(a.out_distances) & 15u) == 0) {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const int64_t idx = static_cast<int32_t>(static_cast<uint32_t>(best[i]));
            oi[i] = idx >= 0 ? idx + index_offset : idx;
        }
        float4* od4 = reinterpret_cast<float4*>(od);
#pragma unroll
        for (int v = 0; v < K / 4; ++v) {
            od4[v] = make_float4(__uint_as_float(static_cast<uint32_t>(best[4 * v] >> 32)),
                                 __uint_as_float(static_cast<uint32_t>(best[4 * v + 1] >> 32)),
                                 __uint_as_float(static_cast<uint32_t>(best[4 * v + 2] >> 32)),
                                 __uint_as_float(static_cast<uint32_t>(best[4 * v + 3] >> 32)));
        }
    } else {
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const int64_t idx = static_cast<int32_t>(static_cast<uint32_t>(best[i]));
            oi[i] = idx >= 0 ? idx + index_offset : idx;
            od[i] = __uint_as_float(static_cast<uint32_t>(best[i] >> 32));
        }
    }
    if constexpr (D > 0 && (K * D) % 4 == 0) {
        if (a.out_positions != nullptr && a.source_cols == D) {
            // Rows of D floats: one load per neighbour, the result row
            // (K * D floats, 16-byte aligned) stored as float4s.
            float row[K * D];
            const SourceRow<D>* src = reinterpret_cast<const SourceRow<D>*>(a.source_points) + pstart;
#pragma unroll
            for (int i = 0; i < K; ++i) {
                const int64_t idx = static_cast<int32_t>(static_cast<uint32_t>(best[i]));
                const SourceRow<D> r = src[idx >= 0 ? idx : 0];
#pragma unroll
                for (int c = 0; c < D; ++c) row[i * D + c] = idx >= 0 ? r.v[c] : 0.0f;
            }
            float4* op = reinterpret_cast<float4*>(a.out_positions + out_row * K * D);
#pragma unroll
            for (int v = 0; v < K * D / 4; ++v) {
                op[v] = make_float4(row[4 * v], row[4 * v + 1], row[4 * v + 2], row[4 * v + 3]);
            }
            return;
        }
    }
    if (a.out_positions != nullptr) {
        const int C = a.source_cols;
        float* op = a.out_positions + out_row * K * C;
#pragma unroll
        for (int i = 0; i < K; ++i) {
            const int64_t idx = static_cast<int32_t>(static_cast<uint32_t>(best[i]));
            const float* src = a.source_points + (pstart + (idx >= 0 ? idx : 0)) * C;
            for (int c = 0; c < C; ++c) op[i * C + c] = idx >= 0 ? src[c] : 0.0f;
        }
    }
}

// Exact distance to a point stored as float4, bit-identical to box_distance
// on the point's degenerate box (lo = hi = p) for every input, NaN and inf
// included.  There, delta = max(p - q, max(0, q - p)); IEEE subtraction is
// sign-symmetric (q - p = -(p - q), also for inf, and NaN for NaN), so
// delta = |p - q| when p - q is not NaN and 0 when it is (max returns the
// non-NaN operand: a NaN query coordinate, or equal infinities, count 0 on
// that axis).  max(|e|, 0) with e = p - q gives exactly that in one
// instruction (abs is a source modifier; arithmetic NaNs are quiet).
template <int D>
__device__ __forceinline__ float point_distance(const float* q, const float4 p) {
    const float pc[3] = {p.x, p.y, p.z};
    float s = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const float e = fmaxf(fabsf(pc[d] - q[d]), 0.0f);
        s = d == 0 ? e * e : __builtin_fmaf(e, e, s);
    }
    return s;
}

// Two parked buckets of 6 (3-D) merged at once: each half sorted by the
// 6-input network, then Batcher's odd-even merge of the two sorted halves
// (the 8 + 8 merge with the padding's comparators removed: 17 exchanges),
// after which sorted rank r is in register kRank12[r].  One merge of 12
// candidates into the list, in place of two merges of 6: at K = 32, 41 +
// 12 + 76 exchanges against 2 x (12 + 6 + 66).
constexpr int kMerge66[17][2] = {{0, 6}, {4, 10}, {4, 6}, {2, 8}, {2, 4}, {8, 6}, {1, 7}, {5, 11}, {5, 7},
                                 {3, 9}, {3, 5}, {9, 7}, {1, 2}, {3, 4}, {5, 8}, {9, 6}, {7, 10}};
constexpr int kRank12[12] = {0, 1, 2, 3, 4, 5, 8, 9, 6, 7, 10, 11};

template <int K>
__device__ __forceinline__ void merge_candidates12(uint64_t (&best)[K], uint64_t (&c)[12]) {
    sort_candidates<6, 0>(c);
    sort_candidates<6, 6>(c);
#pragma unroll
    for (int s = 0; s < 17; ++s) key_exchange(c[kMerge66[s][0]], c[kMerge66[s][1]]);
    constexpr int m = K < 12 ? K : 12;
    constexpr MergePlan<K, m> plan{};
#pragma unroll
    for (int i = 0; i < m; ++i) best[K - m + i] = key_min(best[K - m + i], c[kRank12[m - 1 - i]]);
#pragma unroll
    for (int s = 0; s < MergePlan<K, m>::kStages; ++s) {
        const int h = K >> (s + 1);
#pragma unroll
        for (int i = 0; i < K; ++i) {
            if ((i & h) == 0 && ((plan.needed[s] >> i) & 1)) key_exchange(best[i], best[i + h]);
        }
        // At K = 32 the scheduler would otherwise start the next stage's
        // exchanges before this one's maxima, holding up to 32 more VGPRs.
        if constexpr (K >= 32) __builtin_amdgcn_sched_barrier(0);
    }
}

// One wave per work-group: measured against 256 threads, -3.5% at cfg2 and
// -14% at cfg5, whose waves differ most in cost (finer-grained balancing
// over the CUs); 128 falls between, 512 is 13-24% slower.
constexpr int kKnnBlock = 64;
constexpr int kXcds = 8;               // MI355X: work-groups are dealt round-robin over 8 XCDs

// The cell-block search's failure lists (launch positions left for the next
// stage) are cut into kXcds * kGridSubLists sub-lists, each with its own
// count, filled by one atomic add per wave.  Work-group b's sub-list is that
// of its XCD share (b % kXcds, as in the tile map) and of the residue of its
// local tile index (b / kXcds) mod kGridSubLists; the next stage's
// work-group b reads chunk (b / kXcds) / kGridSubLists of the same
// sub-list, so that it takes failures of tiles near its own.  One count per
// XCD share measured 375 us for the first pass at cfg3, where every wave
// fails at once: same-address atomics serialise (about 90 ns each).  The
// counts lie kCountStride words apart, each on a 128-byte line of its own.
constexpr int kGridSubLists = 64;
constexpr int kCountStride = 32;
constexpr int kGridCounts = kXcds * kGridSubLists;  // per list
__device__ __forceinline__ int grid_sublist() {
    return static_cast<int>(blockIdx.x % kXcds) * kGridSubLists + static_cast<int>(blockIdx.x / kXcds) % kGridSubLists;
}
__device__ __forceinline__ int64_t grid_chunk_start() {
    return static_cast<int64_t>(blockIdx.x / kXcds / kGridSubLists) * kKnnBlock;
}

// Entries of a lane's deferred-node stack, all in LDS (6 bytes each: a
// 32-bit child ref and a 16-bit distance, in columns of stride kKnnBlock):
// as many as the LDS budget of each (D, k) holds.  7.5 KB per work-group for
// 3-D k = 16 and 10 KB for 3-D k = 32, the budgets measured best for the
// earlier 8-byte entries (a 17-entry ring at 3-D k = 16 measured +13%
// traversal at cfg2: resume walks); 2-D k = 8 (cfg4) takes 13 entries, 5
// KB, so that 8 one-wave work-groups fit per SIMD (see knn_waves_per_simd;
// cfg4 traversal with 17 / 15 / 13 entries at 6 / 7 / 8 waves: 0.965 /
// 0.935 / 0.920 ms); 6 KB otherwise.
template <int D, int K>
constexpr int lds_stack_entries() {
    if (D == 2 && K == 8) return 13;
    if (D == 3 && K >= 32) return 26;
    if (D == 3 && K >= 16) return 20;
    return 16;
}

// Waves per SIMD the compiler must leave room for (at most 512 / waves
// VGPRs per lane), where the LDS ring allows that many and the kernel fits
// without spilling: 2-D k = 8 fits 64 VGPRs, so 8 waves (cfg4 traversal
// 1.115 -> 0.920 ms with the 13-entry ring, together with the unclamped
// bucket loads).  Elsewhere the compiler's own
// choice: capping 3-D k = 16 at 80 measured +2% at cfg2 (the ring's LDS
// holds it at 5 waves anyway), and 3-D k = 32 spills at 128.
template <int D, int K, bool kCompact>
constexpr int knn_waves_per_simd() {
    return D == 2 && K == 8 ? 8 : kCompact && D == 3 && K == 16 ? 6 : 1;
}

// Bounded deferred-node stack of one lane: a ring of L entries in LDS.  An
// entry is a child ref and its cached box distance truncated to the top 16
// bits of the float (a lower bound: truncation rounds a non-negative float
// down), which is all pruning needs; a popped node that survives it is
// evaluated exactly.  A push onto a full ring drops the oldest entry (the
// far child of the shallowest pending ancestor, pushed while the k-th
// distance was loosest, so the likeliest to be pruned by the time it would
// be popped) and keeps the smallest dropped distance in `lost_min`.
// Nothing is lost for correctness: when the ring empties with lost_min <=
// the k-th distance, the traversal resumes through the parent links (see
// traverse).
//
// Two layouts.  Full (6 bytes per entry): the 32-bit ref in `refs`, the
// distance in `dists`.  Compact (5 bytes; accel clouds of at most
// kCompactCloud points): the ref as a 24-bit code, an internal node as its
// index and a bucket as 1 << 23 | (count - 1) << 20 | first, with the
// distance and the code's low 16 bits in one word of `refs` and its high 8
// bits in `hi`.  At 3-D k = 16 the compact ring's 20 entries take 6.4 KB,
// so 6 work-groups fit per SIMD instead of 5 (cfg2 traversal -2.6%, cfg3
// -1.4%).
constexpr int64_t kCompactCloud = int64_t(1) << 20;

template <int L, bool kCompact>
struct RingStack {
    uint32_t* refs;   // this lane's column: slot i at refs[i * kKnnBlock]
    uint16_t* dists;  // full layout, likewise
    uint8_t* hi;      // compact layout, likewise
    int top = 0;      // slot of the next push
    int count = 0;
    float lost_min = INFINITY;

    __device__ __forceinline__ static uint32_t encode(int32_t ref) {
        const uint32_t r = static_cast<uint32_t>(ref);
        return ref < 0 ? 0x800000u | (((r >> 28) & 7u) << 20) | (r & 0xFFFFFu) : r;
    }
    __device__ __forceinline__ static int32_t decode(uint32_t c) {
        return (c & 0x800000u) ? static_cast<int32_t>(0x80000000u | (((c >> 20) & 7u) << 28) | (c & 0xFFFFFu))
                                : static_cast<int32_t>(c);
    }
    __device__ __forceinline__ float dist_at(int slot) const {
        if constexpr (kCompact) return __uint_as_float(refs[slot * kKnnBlock] & 0xFFFF0000u);
        else return __uint_as_float(static_cast<uint32_t>(dists[slot * kKnnBlock]) << 16);
    }
    __device__ __forceinline__ void push(float d, int32_t ref) {
        if (count == L) {
            // Full: slot `top` holds the oldest entry.
            lost_min = fminf(lost_min, dist_at(top));
        } else {
            ++count;
        }
        if constexpr (kCompact) {
            const uint32_t c = encode(ref);
            refs[top * kKnnBlock] = (__float_as_uint(d) & 0xFFFF0000u) | (c & 0xFFFFu);
            hi[top * kKnnBlock] = static_cast<uint8_t>(c >> 16);
        } else {
            refs[top * kKnnBlock] = static_cast<uint32_t>(ref);
            dists[top * kKnnBlock] = static_cast<uint16_t>(__float_as_uint(d) >> 16);
        }
        top = top == L - 1 ? 0 : top + 1;
    }
    __device__ __forceinline__ void read(int slot, float& d, int32_t& ref) const {
        if constexpr (kCompact) {
            const uint32_t w = refs[slot * kKnnBlock];
            ref = decode((static_cast<uint32_t>(hi[slot * kKnnBlock]) << 16) | (w & 0xFFFFu));
            d = __uint_as_float(w & 0xFFFF0000u);
        } else {
            ref = static_cast<int32_t>(refs[slot * kKnnBlock]);
            d = __uint_as_float(static_cast<uint32_t>(dists[slot * kKnnBlock]) << 16);
        }
    }
    // Pop with a one-entry look-ahead: the top two entries are read together
    // and the top one, if already beyond `worst` (the k-th distance, which
    // would prune it at the next test), is dropped in the same step.  The
    // same entries are discarded as by popping twice, one loop iteration
    // sooner.  Used by the 2-D traversals, where pruned pops take 19% of the
    // lane slots at cfg4 (traversal -1.6%; +2.3% at cfg5 in 3-D, not used).
    __device__ __forceinline__ void pop_lookahead(float& d, int32_t& ref, float worst) {
        const int t1 = top == 0 ? L - 1 : top - 1;
        const int t2 = t1 == 0 ? L - 1 : t1 - 1;
        float d1, d2;
        int32_t r1, r2;
        read(t1, d1, r1);
        read(t2, d2, r2);
        const bool skip = count >= 2 && !(d1 <= worst);
        top = skip ? t2 : t1;
        count -= skip ? 2 : 1;
        d = skip ? d2 : d1;
        ref = skip ? r2 : r1;
    }
    __device__ __forceinline__ void pop(float& d, int32_t& ref) {
        top = top == 0 ? L - 1 : top - 1;
        --count;
        if constexpr (kCompact) {
            const uint32_t w = refs[top * kKnnBlock];
            ref = decode((static_cast<uint32_t>(hi[top * kKnnBlock]) << 16) | (w & 0xFFFFu));
            d = __uint_as_float(w & 0xFFFF0000u);
        } else {
            ref = static_cast<int32_t>(refs[top * kKnnBlock]);
            d = __uint_as_float(static_cast<uint32_t>(dists[top * kKnnBlock]) << 16);
        }
    }
};

// ---------------------------------------------------------------------------
// Node sources.  The traversal reaches a structure only through these
// members: `root()`, `is_bucket(ref)`, `is_internal(ref)`, `children(ref,
// ...)` (both child box distances and refs; an absent child has distance
// +inf, which no k-th distance admits), `parent(ref)` (-1 above the root)
// and `scan(bucket, ...)` (brute force of a bucket's points into the
// candidate list), plus `kNone`, a ref that is never a bucket.
// ---------------------------------------------------------------------------

// The acceleration structure (accel.hip): an internal node's record holds
// both child boxes, both child refs and its parent; a bucket (negative ref:
// first position in the low 28 bits, count - 1 in bits 28-30) is up to
// accel_bucket<D>() consecutive Morton-ordered points, loaded together.
//
// With kRows, `pts` and `recs` point at the call's first cloud (one address
// for the whole launch, held in scalar registers) and `first_row` locates
// this cloud; without it they point at this cloud (two 64-bit addresses per
// lane, and no add per access).  3-D k = 32 takes kRows: with the merges'
// stage barriers it then fits 126 VGPRs, 4 waves per SIMD instead of 3
// (cfg5 traversal 20.26 -> 17.89 ms); elsewhere kRows measured +1% (cfg2,
// cfg3) at unchanged occupancy.
template <int D, bool kRows>
struct AccelNodes {
    static constexpr int kDims = D;
    static constexpr int R = 4 * D + 4;
    static constexpr int32_t kNone = 0;  // bucket refs are negative
    const float4* pts;                   // points (see above)
    const float* recs;                   // record rows
    int first_row;                       // kRows: this cloud's first row (rows fit in int32)
    int n;

    __device__ __forceinline__ int64_t row(int r) const {
        return kRows ? static_cast<int64_t>(first_row + r) : static_cast<int64_t>(r);
    }

    __device__ __forceinline__ int32_t root() const {
        return n <= accel_bucket<D>() ? static_cast<int32_t>(0x80000000u | (static_cast<uint32_t>(n - 1) << 28))
                                      : 0;
    }
    __device__ __forceinline__ bool is_bucket(int32_t ref) const { return ref < 0; }
    __device__ __forceinline__ bool is_internal(int32_t ref) const { return ref < n - 1; }

    __device__ __forceinline__ void children(int32_t ref, const float* q, float& ld, float& rd, int32_t& lref,
                                             int32_t& rref) const {
        const float4* r4 = reinterpret_cast<const float4*>(recs + row(ref) * R);
        float rec[R];
#pragma unroll
        for (int v = 0; v < R / 4; ++v) {
            const float4 x = r4[v];
            rec[4 * v] = x.x;
            rec[4 * v + 1] = x.y;
            rec[4 * v + 2] = x.z;
            rec[4 * v + 3] = x.w;
        }
        ld = box_distance<D>(q, rec);
        rd = box_distance<D>(q, rec + 2 * D);
        lref = __float_as_int(rec[4 * D]);
        rref = __float_as_int(rec[4 * D + 1]);
    }

    // An internal node's parent is in its own row; a bucket's, in the last
    // word of the row where it starts; -1 above the root.  A ref outside the
    // cloud is not read, and it or a stored link outside the cloud's
    // internal nodes (neither of which a well-formed accel holds) returns
    // kCorruptLink.
    static constexpr int32_t kCorruptLink = -2;
    __device__ __forceinline__ int32_t parent(int32_t ref) const {
        if (ref == root()) return -1;
        const int first = ref & 0x0fffffff;
        if (ref >= 0 ? ref >= n - 1 : first + ((ref >> 28) & 7) + 1 > n) return kCorruptLink;
        const int32_t par = __float_as_int(recs[row(ref >= 0 ? ref : first) * R + 4 * D + (ref >= 0 ? 2 : 3)]);
        return par >= 0 && par < n - 1 ? par : kCorruptLink;
    }

    template <int K>
    __device__ __forceinline__ void scan(int32_t ref, const float* q, uint64_t (&best)[K]) const {
        const int first = ref & 0x0fffffff;
        const int count = ((ref >> 28) & 7) + 1;
        // Only an accel this library did not build for these clouds holds
        // such a ref (the Python layer refuses any other pairing; the C ABI
        // states it as a precondition): nothing outside the cloud is read.
        // Marking the row instead measured +27 VGPRs at 3-D k = 32 (a wave
        // per SIMD less) and spills at 3-D k = 16, so the row is left as
        // the traversal found it.
        if (first + count > n) return;
        constexpr int kBucket = accel_bucket<D>();
        // Every slot loads, so the loads issue together from one address.
        // Slots past the bucket (masked below) read at most kBucket - 1 rows
        // past `first + count - 1 < n`: the next cloud's points or, after the
        // last cloud, the points area's padding to 256 bytes and the record
        // rows behind it (>= 48 bytes per point), so every read stays inside
        // the accel buffer (accel_bytes).
        const float4* b = pts + row(first);
        float4 p[kBucket];
#pragma unroll
        for (int j = 0; j < kBucket; ++j) p[j] = b[j];
        // The loads issue at the traversal's priority; the merge runs at 0.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(0);
        uint64_t c[kBucket];
#pragma unroll
        for (int j = 0; j < kBucket; ++j) {
            const float d = point_distance<D>(q, p[j]);
            c[j] = j < count && d < kFar ? candidate_key(d, __float_as_uint(p[j].w)) : kEmptyKey;
        }
        merge_candidates<K, kBucket>(best, c);
    }

    // Both parked buckets of a lane in one merge (3-D: 6 + 6 candidates);
    // `ref2` is kNone when the lane holds one.
    template <int K>
    __device__ __forceinline__ void scan2(int32_t ref1, int32_t ref2, const float* q, uint64_t (&best)[K]) const {
        static_assert(accel_bucket<D>() == 6, "two-bucket merges are for 6-point buckets");
        uint64_t c[12];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int32_t ref = b == 0 ? ref1 : ref2;
            int first = ref & 0x0fffffff;
            int count = ((ref >> 28) & 7) + 1;
            if (ref == kNone || first + count > n) {
                first = 0;  // absent, or a corrupt ref: no candidates
                count = 0;
            }
            // Past the bucket: rows inside the accel buffer, as in scan.
            const float4* rows = pts + row(first);
            float4 p[6];
#pragma unroll
            for (int j = 0; j < 6; ++j) p[j] = rows[j];
#pragma unroll
            for (int j = 0; j < 6; ++j) {
                const float d = point_distance<D>(q, p[j]);
                c[6 * b + j] = j < count && d < kFar ? candidate_key(d, __float_as_uint(p[j].w)) : kEmptyKey;
            }
        }
        merge_candidates12<K>(best, c);
    }
};

// The reference's implicit tree (implicit_tree.cuh:26-127): refs are heap
// indices, a node's children are 2i + 1 and 2i + 2 (the right one possibly
// virtual) and its parent (i - 1) / 2.  The "buckets" are the leaves'
// parents (level L - 1; the root when it is the only leaf): their scan
// scores both leaves from their own (degenerate) boxes with box_distance,
// exactly as the reference scores a leaf, near leaf first, each against the
// k-th distance as it stands then; that is the reference's visit of the two
// leaves (the far leaf is pushed, the near one entered, and the far one
// popped straight after), with no stack entry.
template <int D>
struct HeapNodes {
    static constexpr int kDims = D;
    static constexpr int32_t kNone = -1;
    const float* nodes;     // this tree's rows of 2 * D floats
    const int64_t* sorted;  // this cloud's sorted indices
    int n;
    int L;                  // leaf level
    int vl;                 // virtual leaves
    int bucket_first;       // heap index of the first node on the leaves' parents' level
    int leaf_row0;          // storage row of leaf position 0

    __device__ __forceinline__ void init(const float* nodes_, const int64_t* sorted_, int n_) {
        nodes = nodes_;
        sorted = sorted_;
        n = n_;
        L = tree::leaf_level(n);
        vl = tree::virtual_leaves(n);
        bucket_first = tree::level_first(L > 0 ? L - 1 : 0);
        leaf_row0 = tree::memory_index(vl, L, tree::level_first(L));
    }
    __device__ __forceinline__ int32_t root() const { return 0; }
    __device__ __forceinline__ bool is_bucket(int32_t ref) const { return ref >= bucket_first; }
    __device__ __forceinline__ bool is_internal(int32_t) const { return true; }

    __device__ __forceinline__ void children(int32_t ref, const float* q, float& ld, float& rd, int32_t& lref,
                                             int32_t& rref) const {
        lref = 2 * ref + 1;
        rref = lref + 1;
        // The real nodes of a level are consecutive rows, so a real right
        // child is the row after the left one.
        const float* box = nodes + static_cast<int64_t>(tree::memory_index(vl, L, lref)) * (2 * D);
        ld = box_distance<D>(q, box);
        rd = tree::is_virtual(vl, L, rref) ? INFINITY : box_distance<D>(q, box + 2 * D);
    }

    __device__ __forceinline__ int32_t parent(int32_t ref) const { return ref > 0 ? (ref - 1) >> 1 : -1; }

    template <int K>
    __device__ __forceinline__ void scan(int32_t ref, const float* q, uint64_t (&best)[K]) const {
        // Leaf positions of the pair (a lone root leaf: position 0 only);
        // the real leaves are positions < n.
        const int p = L > 0 ? 2 * ref + 1 - tree::level_first(L) : 0;
        const bool right_real = L > 0 && p + 1 < n;
        const float* box = nodes + static_cast<int64_t>(leaf_row0 + p) * (2 * D);
        const float ld = box_distance<D>(q, box);
        const float rd = right_real ? box_distance<D>(q, box + 2 * D) : INFINITY;
        const bool left_near = ld <= rd;
        const int near_p = left_near ? p : p + 1;
        const float near_d = left_near ? ld : rd;
        const uint64_t near_key = candidate_key(near_d, static_cast<uint32_t>(sorted[near_p]));
        if (near_d < kFar && near_key < best[K - 1]) insert_sorted<K>(best, near_key);
        if (right_real) {
            const int far_p = left_near ? p + 1 : p;
            const float far_d = left_near ? rd : ld;
            const uint64_t far_key = candidate_key(far_d, static_cast<uint32_t>(sorted[far_p]));
            if (far_d < kFar && far_key < best[K - 1]) insert_sorted<K>(best, far_key);
        }
    }
};

// Branch-and-bound of one query over a node source: the reference's pruning
// rule, near-first order (ties to the left child) and cached far-child
// distances, with a bounded stack and postponed bucket scans.
//
// Bounded stack, exact resume.  The stack is a ring of lds_stack_entries
// entries in LDS (RingStack); nothing lives in scratch.  When a push drops
// the oldest entry, the lane records the smallest dropped distance.  When
// the ring runs empty, nothing dropped can matter if that distance exceeds
// the k-th distance (which only shrinks), and the lane is done.  Otherwise
// it walks up from the last node it entered through the parent links: at
// each ancestor it recomputes the two child distances, and if it came up
// from the near child and the far child is within the k-th distance, the
// far child is still pending (it was dropped: a far child pushed and not
// dropped is popped before the ring empties, after which the walk comes up
// through it) and the traversal resumes there; otherwise it goes on up, and
// at the root it is done.  The walk recomputes the same near/far choice the
// descent made (same query, same boxes, ties to the left), so no subtree is
// entered twice and no candidate is inserted twice.  Nor does the ring
// change the order of visits: the dropped entries are the bottom of the
// stack, which an unbounded stack would also pop last, deepest first, and
// the walk reaches them in that order and tests each with its exact
// distance; a popped entry whose truncated distance passes but whose exact
// one would not is entered and finds both children beyond the k-th distance
// (a child's box lies inside its parent's, so its distance is no smaller),
// as if it had been pruned.  A walk step over the
// accel costs two dependent loads (the parent link, then the parent's
// record), and one walking lane holds up its wave, so the ring is sized to
// make drops rare: a CPU model of the accel traversal at cfg2 showed no
// query deeper than 21 entries (a 16-entry ring of 8-byte entries made
// every query drop and measured +20% traversal time).
//
// Postponed buckets.  With one query per lane, scoring a bucket and merging
// its candidates into the sorted list (merge_candidates: a fixed network of
// O(K log K) min/max) is the dominant cost, and the wave pays for it
// whenever any lane scans.  So a lane that reaches a bucket parks it and
// keeps traversing; a lane that reaches a bucket while it holds one waits
// (one parked bucket per lane: two measured 2% slower at k = 8 and no
// better at k >= 16, with one insertion per candidate).
// At the loop head, which every lane of the wave passes each iteration, the
// wave scans all parked buckets together once at least half of its live
// lanes hold one, or no lane can move: the merges then run with most lanes
// active.  Meanwhile a lane prunes with its list's current k-th distance, a
// valid (looser) bound, and a waiting lane re-tests its bucket after the
// round, so results are unchanged; the end result is the k smallest
// (distance, index) pairs whatever the order of visits.  Measured on MI355X
// over the accel against immediate insertion (one insertion per accepted
// candidate, then): -20% at k = 16 (cfg2), -13% at k = 8 (cfg4); a variant
// that buffered candidates in LDS and merged them wave-wide with sorting
// networks was slower (fewer waves fit).  The per-lane merge network in
// place of one insertion per candidate: traversal -12% at cfg2, cfg3 and
// cfg4, -6% at cfg5 (k = 32).  3-D k = 32 parks two buckets per lane and
// merges their 12 candidates at once (merge_candidates12), flushing when a
// quarter of the live lanes hold two: half the flushes and 129 exchanges per
// 12 candidates instead of 168; cfg5 traversal 22.5 -> 20.4 ms (both at 3
// waves per SIMD).  At k = 16 two slots measured +1.5-2% (cfg2, cfg3).
//
// Without kPostpone, buckets are scanned when reached, so the traversal makes
// the reference's visits in the reference's order.  The implicit tree runs
// that way: where the result does depend on the order (points with a NaN
// coordinate, whose distances the node boxes do not bound), it is then the
// reference's result.
template <bool kPostpone, int K, int L, bool kCompact, class Nodes>
__device__ __forceinline__ void traverse(const Nodes& t, const float* q, uint64_t (&best)[K],
                                         RingStack<L, kCompact>& stack) {
    // 3-D k = 32 parks two buckets per lane and merges them together.
    constexpr bool kTwoSlots = kPostpone && K >= 32 && Nodes::kDims == 3;
    int32_t ref = t.root();
    float nd = 0.0f;
    int32_t parked = Nodes::kNone;
    int32_t parked2 = Nodes::kNone;
    bool waiting = false;
    bool done = false;

    // Wave priority: between flushes a wave runs a chain of dependent record
    // loads (visit, push, pop), and its next load should issue as soon as
    // the last one returns; a flush's merges are a long VALU run that can
    // yield.  So the traversal runs at priority 1 and a scan drops to 0 once
    // its bucket loads are issued, until the flush ends (traversal -5% at
    // cfg2, -3% at cfg3 and cfg5, -1% at cfg4; 1 and 3 measured the same).
    if constexpr (kPostpone) __builtin_amdgcn_s_setprio(1);
    // Descents `continue` straight to the loop head; this shape keeps them
    // in a tight loop (a flag-driven single loop of the same work measured
    // 2x slower).
    while (true) {
        // Not in a scope of its own: a block here (an `if constexpr` body)
        // reorders the loop's blocks and measured +5% traversal time.
        const uint64_t holding = kPostpone ? __ballot(parked != Nodes::kNone) : 0;
        if (holding != 0) {
            const uint64_t live = __ballot(true);
            const uint64_t movable = __ballot(!waiting && !done);
            const uint64_t full = kTwoSlots ? __ballot(parked2 != Nodes::kNone) : holding;
            // One slot: flush once half the live lanes hold a bucket; two
            // slots: once a quarter of them hold two (cfg5 traversal at 4
            // waves per SIMD with 3/8, 1/4, 3/16, 1/8: 18.15, 17.90, 18.26,
            // 18.85 ms; at 3 waves 1/2 had measured 21.3 against 20.4).
            constexpr int kNum = 1, kDen = kTwoSlots ? 4 : 2;
            if (movable == 0 || kNum * __popcll(live) <= kDen * __popcll(full)) {
                // One slot: the scan drops the priority once its loads are
                // issued; two slots (k = 32) drop it here (inside the
                // two-bucket scan the drop cost the fourth wave per SIMD:
                // cfg5 +13%).
                if constexpr (kTwoSlots) __builtin_amdgcn_s_setprio(0);
                if (parked != Nodes::kNone) {
                    if constexpr (kTwoSlots) t.scan2(parked, parked2, q, best);
                    else t.scan(parked, q, best);
                }
                parked = Nodes::kNone;
                parked2 = Nodes::kNone;
                waiting = false;
                __builtin_amdgcn_s_setprio(1);
            }
        }
        if (done) {
            if (parked == Nodes::kNone) break;
            continue;
        }
        if (waiting) continue;
        const float worst = __uint_as_float(static_cast<uint32_t>(best[K - 1] >> 32));
        if (nd <= worst) {
            if (t.is_bucket(ref)) {
                if constexpr (kPostpone) {
                    // Park the bucket; a lane whose slots are taken waits and
                    // revisits this bucket after the next round.
                    if (parked == Nodes::kNone) {
                        parked = ref;
                    } else if (kTwoSlots && parked2 == Nodes::kNone) {
                        parked2 = ref;
                    } else {
                        waiting = true;
                        continue;
                    }
                } else {
                    t.scan(ref, q, best);
                }
            } else if (t.is_internal(ref)) {
                float ld, rd;
                int32_t lref, rref;
                t.children(ref, q, ld, rd, lref, rref);
                const bool left_near = ld <= rd;
                const int32_t near_ref = left_near ? lref : rref;
                const int32_t far_ref = left_near ? rref : lref;
                const float near_d = left_near ? ld : rd;
                const float far_d = left_near ? rd : ld;
                if (far_d <= worst) stack.push(far_d, far_ref);
                if (near_d <= worst) {
                    ref = near_ref;
                    nd = near_d;
                    continue;
                }
            }
        }
        if (stack.count == 0) {
            if (!(stack.lost_min <= worst)) {
                done = true;  // stays in the loop until its parked buckets are scanned
                continue;
            }
            // One step of the resume walk from `ref`, the last node entered
            // (its subtree is finished), to its parent.
            const int32_t par = t.parent(ref);
            if (par < 0) {
                done = true;
                continue;
            }
            float ld, rd;
            int32_t lref, rref;
            t.children(par, q, ld, rd, lref, rref);
            const bool left_near = ld <= rd;
            const int32_t near_ref = left_near ? lref : rref;
            const int32_t far_ref = left_near ? rref : lref;
            const float far_d = left_near ? rd : ld;
            if (ref == near_ref && far_d <= worst) {
                ref = far_ref;  // a dropped far child: resume there
                nd = far_d;
            } else {
                ref = par;  // finished here too: next step from the parent
                nd = INFINITY;
            }
            continue;
        }
        if constexpr (Nodes::kDims == 2) stack.pop_lookahead(nd, ref, worst);
        else stack.pop(nd, ref);
    }
    if constexpr (kPostpone) __builtin_amdgcn_s_setprio(0);
}

// One query per lane over the implicit tree (kAccel false) or the accel;
// the body of both kernels below.
//
// Tile order: consecutive work-groups land on different XCDs, each with its
// own L2; logical tile t = (block % 8) * (grid / 8) + block / 8 gives every
// XCD a contiguous run of Morton-ordered queries, so one XCD's L2 serves a
// compact region of the tree.
// Where query `gid` of the launch reads and writes: its cloud, its input row
// and output row, and the structure it searches.
struct QueryLoc {
    int64_t row;           // input row (queries), -1 for a corrupt order entry
    int64_t out_row;       // result row
    int64_t pstart;        // the cloud's first point row
    int64_t nstart;        // the cloud's first node row (implicit tree)
    int64_t index_offset;  // added to result indices (false route)
    int n;                 // the cloud's points
    bool second;           // false route: the second structure
};

template <bool kOrdered, bool kRagged, bool kRouted, bool kAccel>
__device__ __forceinline__ QueryLoc locate(const KnnArgs& a, int64_t gid) {
    QueryLoc l;
    int64_t seg, qbase, qcount;
    if constexpr (kRagged) {
        seg = find_segment([&](int i) { return a.query_offsets[i]; }, static_cast<int>(a.B), gid);
        qbase = a.query_offsets[seg];
        qcount = a.query_offsets[seg + 1] - qbase;
        l.pstart = a.point_offsets[seg];
        l.n = static_cast<int>(a.point_offsets[seg + 1] - l.pstart);
        l.nstart = kAccel ? 0 : a.node_offsets[seg];
    } else {
        seg = gid / a.M;
        qbase = seg * a.M;
        qcount = a.M;
        l.n = a.num_leaves;
        l.pstart = seg * static_cast<int64_t>(l.n);
        l.nstart = seg * static_cast<int64_t>(a.num_real_nodes);
    }
    const int64_t local = gid - qbase;
    const int64_t qi = kOrdered ? a.order[qbase + local] : local;
    l.row = qi < 0 || qi >= qcount ? -1 : qbase + qi;  // a corrupt order never indexes out of range
    // Spatial output (knn_query.cu:147-148) keeps the launch (Morton) order.
    l.out_row = a.spatial_output ? gid : l.row;
    l.second = false;
    l.index_offset = 0;
    if (kRouted && l.row >= 0 && a.routes[l.row] == 0) {
        // False route (knn_query.cu:205-217): the second structure, indices
        // after the first's points.
        l.second = true;
        l.index_offset = l.n;
        l.n = a.num_leaves2;
        l.pstart = seg * static_cast<int64_t>(l.n);
        l.nstart = seg * static_cast<int64_t>(a.num_real_nodes2);
    }
    return l;
}

template <int D, int K, bool kOrdered, bool kRagged, bool kRouted, bool kAccel, bool kCompact>
__device__ __forceinline__ void knn_query(const KnnArgs& a) {
    constexpr int kLds = lds_stack_entries<D, K>();
    __shared__ uint32_t lds_refs[kLds * kKnnBlock];
    __shared__ uint16_t lds_dists[kCompact ? 1 : kLds * kKnnBlock];
    __shared__ uint8_t lds_hi[kCompact ? kLds * kKnnBlock : 1];
    const int64_t per_xcd = gridDim.x / kXcds;
    // The cell-block search's fallback pass: its list names the launch
    // positions left to search, and bounds the k-th distance of each (at
    // least k points lie within it, so slots seeded (bound, 0xffffffff) are
    // all displaced by points, the bound's own included: the result is
    // exact).  Work-group b takes a chunk of sub-list grid_sublist(), fb_seg
    // entries apart (the grid is sized for every query).
    const bool fallback = kAccel && a.fb_list != nullptr;
    const int64_t tile = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    int64_t gid = tile * kKnnBlock + threadIdx.x;
    float seed = kFar;
    if (fallback) {
        const int64_t listed = a.fb_count[grid_sublist() * kCountStride];
        const int64_t at = grid_chunk_start() + threadIdx.x;
        if (at >= listed) return;
        gid = a.fb_list[grid_sublist() * a.fb_seg + at];
        seed = a.fb_bound[gid];
    }
    if (gid >= a.total_q) return;
    const QueryLoc in = locate<kOrdered, kRagged, kRouted, kAccel>(a, gid);
    if (in.row < 0) return;

    float q[D];
#pragma unroll
    for (int d = 0; d < D; ++d) q[d] = a.queries[in.row * D + d];

    uint64_t best[K];
#pragma unroll
    for (int i = 0; i < K; ++i) best[i] = candidate_key(seed, 0xffffffffu);

    RingStack<kLds, kCompact> stack;
    stack.refs = lds_refs + threadIdx.x;
    stack.dists = lds_dists + (kCompact ? 0 : threadIdx.x);
    stack.hi = lds_hi + (kCompact ? threadIdx.x : 0);
    if constexpr (kAccel) {
        const void* accel = in.second ? a.accel2 : a.accel;
        const int64_t total_points = in.second ? a.B * static_cast<int64_t>(in.n) : a.total_points;
        constexpr bool kRows = K >= 32;
        AccelNodes<D, kRows> t;
        const float4* pts = static_cast<const float4*>(accel);
        const float* recs =
            reinterpret_cast<const float*>(static_cast<const char*>(accel) + accel_points_bytes(total_points));
        t.pts = kRows ? pts : pts + in.pstart;
        t.recs = kRows ? recs : recs + in.pstart * AccelNodes<D, kRows>::R;
        t.first_row = kRows ? static_cast<int>(in.pstart) : 0;
        t.n = in.n;
        traverse<true>(t, q, best, stack);
    } else {
        HeapNodes<D> t;
        t.init((in.second ? a.node_aabbs2 : a.node_aabbs) + in.nstart * 2 * D,
               (in.second ? a.sorted_indices2 : a.sorted_indices) + in.pstart, in.n);
        traverse<false>(t, q, best, stack);
    }

    // The output location is derived again from the lane's position (the
    // work-group is one wave, so the lane id is threadIdx.x) instead of being
    // held in registers through the traversal: the compiler cannot tell the
    // two apart, so nothing of the first derivation stays live.
    int64_t gid_out = tile * kKnnBlock + __lane_id();
    if (fallback) gid_out = a.fb_list[grid_sublist() * a.fb_seg + grid_chunk_start() + __lane_id()];
    const QueryLoc out = locate<kOrdered, kRagged, kRouted, kAccel>(a, gid_out);
    write_results<K, D>(a, out.out_row, best, out.index_offset, out.pstart);
}

// Separate names, so profiles tell the two traversals apart.
// The routed traversal (two structures, chosen per query) has kernels of its
// own, so the plain ones carry none of its per-lane state.
template <int D, int K, bool kOrdered, bool kRagged, bool kRouted>
__global__ __launch_bounds__(kKnnBlock) void knn_kernel(KnnArgs a) {
    knn_query<D, K, kOrdered, kRagged, kRouted, false, false>(a);
}

template <int D, int K, bool kOrdered, bool kRagged, bool kRouted, bool kCompact>
__global__ __launch_bounds__(kKnnBlock) __attribute__((amdgpu_waves_per_eu(knn_waves_per_simd<D, K, kCompact>()))) void
knn_accel_kernel(KnnArgs a) {
    knn_query<D, K, kOrdered, kRagged, kRouted, true, kCompact>(a);
}

// ---------------------------------------------------------------------------
// Cell-block search (batched accel calls, near-uniform clouds).
//
// The accel's points are in Morton order, so the points of any level-l
// Morton cell (the code's top D*l bits) are one contiguous run of them;
// `table` holds each cell's first point (cell c's run is [table[c],
// table[c + 1])).  A query scans the 3^D cells around its own (its
// coordinates quantised as the points' were) and merges their points into
// its list with the bucket merge.  Every point outside the block lies
// beyond the block's boundary, at least `margin` from the query; when the
// list's k-th distance is below margin^2 no such point can enter it, so the
// list is the exact result, bit for bit (the same k smallest (distance,
// index) keys).  The margin is taken short of the boundary by 1e-5 of the
// larger of the box's extents and its coordinates' magnitudes: the rounding
// of the quantisation (x - lo, the division), of the boundary and of the
// distances adds up to about 5e-7 of that, and the squared distances keep
// the strict order with the rest.  Queries that fail (or find the block too
// full, or whose cloud the table kernel disabled) go to the accel traversal
// with the block's k-th distance as the starting bound.  Measured on MI355X
// (k-NN call, same inputs, cell-block path against the traversal alone):
// cfg2 0.58 -> 0.43 ms (scan 0.25, fallback over 13% of the queries 0.12,
// table and list 0.02), 3-D k = 8 0.54 -> 0.34, cfg4 0.92 -> 0.68, 2-D
// k = 32 2.00 -> 1.53, 3-D k = 32 0.97 -> 0.94, cfg3 (clouds disabled:
// long empty runs) 1.16 -> 1.17 ms.
// ---------------------------------------------------------------------------
template <int D>
constexpr int grid_axis_bits() { return D == 3 ? 10 : 16; }

template <int D>
__device__ __forceinline__ uint32_t grid_cell_id(const uint32_t (&c)[D]) {
    if constexpr (D == 3) return morton::spread3(c[0]) | (morton::spread3(c[1]) << 1) | (morton::spread3(c[2]) << 2);
    else return morton::spread2(c[0]) | (morton::spread2(c[1]) << 1);
}

// The level-l cell of a point (or query) against the cloud's box: the top l
// bits of each axis of its Morton cell, so the cell id is its code >>
// (D * (axis bits - l)).
template <int D>
__device__ __forceinline__ void grid_cell(const float* p, const float* lo, const float* hi, int shift,
                                          uint32_t (&c)[D]) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
        c[d] = morton::cell(morton::unit_coord(p[d], lo[d], hi[d]), 1u << grid_axis_bits<D>()) >> shift;
    }
}

// Longest run of empty cells (in Morton order) a cloud may have: a longer
// one means a large empty region, so the cloud is not near-uniform and the
// block search is off for it (at the levels chosen, a uniform cloud has one
// with probability below 1e-14).
constexpr int kGridMaxGap = 64;

// Clears the clouds' flags and the failure lists' counts (`ncounts` of
// them, kCountStride words apart).
__global__ void grid_init_kernel(uint32_t* flags, int64_t B, uint32_t* counts, int ncounts) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < B) flags[i] = 0u;
    if (i < ncounts) counts[i * kCountStride] = 0u;
}

// Appends the lanes set in `left` (wave-uniform) to this work-group's
// sub-list of a failure list (`seg` entries each).  A sub-list holds the
// launch positions of one residue class of one XCD share's tiles (or, for
// the second list, of one sub-list of the first), at most `seg` of them,
// so it cannot overflow.  One atomic per wave reserves the entries; their
// order within a sub-list follows the waves' completion and changes no
// result (each query's search depends only on the query and its bound).
__device__ __forceinline__ void grid_append(int32_t* list, uint32_t* counts, int64_t seg, uint64_t left,
                                            int64_t gid) {
    if (left == 0) return;
    const int sub = grid_sublist();
    // The first active lane reserves the entries and hands out the base.
    const int leader = __ffsll(static_cast<long long>(__ballot(1))) - 1;
    uint32_t base = 0;
    if (lane_id() == leader) base = atomicAdd(&counts[sub * kCountStride], static_cast<uint32_t>(__popcll(left)));
    base = __builtin_amdgcn_readlane(base, leader);
    if ((left >> lane_id()) & 1ull) {
        const uint32_t rank = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(left >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(left), 0u));
        list[sub * seg + base + rank] = static_cast<int32_t>(gid);
    }
}

// One thread per point: writes the first-point entries of the cells from the
// previous point's cell (exclusive) to its own, and after the last point
// those up to the end.  flags[b] = 1 disables cloud b: a non-finite point or
// box, an empty extent, a cell order that does not follow the points' (the
// box is not the one their codes were taken against), or an empty run
// longer than kGridMaxGap (its entries are then left unwritten, and unread).
template <int D>
__global__ __launch_bounds__(kBlock) void grid_table_kernel(const float4* __restrict__ pts,
                                                            const float* __restrict__ node_aabbs, int64_t nr, int64_t B,
                                                            int n, int level, int32_t* __restrict__ table,
                                                            uint32_t* __restrict__ flags) {
    // B * n fits in int32 (the entry points check it).
    const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= B * n) return;
    const int b = i / n;
    const int j = i - b * n;
    const float* root = node_aabbs + b * nr * 2 * D;
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        lo[d] = root[d];
        hi[d] = root[D + d];
    }
    const int shift = grid_axis_bits<D>() - level;
    const int64_t cells = int64_t(1) << (D * level);
    int32_t* t = table + static_cast<int64_t>(b) * (cells + 1);
    auto cell_of = [&](int64_t r, bool& ok) {
        const float4 p4 = pts[r];
        const float p[3] = {p4.x, p4.y, p4.z};
        uint32_t c[D];
        grid_cell<D>(p, lo, hi, shift, c);
#pragma unroll
        for (int d = 0; d < D; ++d) ok = ok && isfinite(p[d]);
        return static_cast<int64_t>(grid_cell_id<D>(c));
    };
    bool ok = true;
    const int64_t own = cell_of(i, ok);
    // The previous point's cell is the previous lane's own (its cloud's, when
    // j > 0), except in lane 0.
    int64_t prev = __shfl_up(own, 1);
    if (j == 0) {
        prev = -1;
    } else if (lane_id() == 0) {
        bool prev_ok = true;
        prev = cell_of(i - 1, prev_ok);
    }
    if (j == 0) {
#pragma unroll
        for (int d = 0; d < D; ++d) ok = ok && isfinite(lo[d]) && isfinite(hi[d]) && hi[d] > lo[d];
    }
    const int64_t last = j == n - 1 ? cells : own;  // after the last point: every cell to the end
    if (!ok || own < prev || own - prev > kGridMaxGap || last - own > kGridMaxGap) {
        flags[b] = 1u;
        return;
    }
    for (int64_t c = prev + 1; c <= own; ++c) t[c] = j;
    for (int64_t c = own + 1; c <= last; ++c) t[c] = n;
}

// The cells of a block of (2W + 1)^D cells as offsets from the query's
// cell, nearest first (by squared offset, then in storage order): its own,
// then (W = 1) those sharing a face with it, an edge, a corner.  Each is
// (dx + W) | (dy + W) << 3 | (dz + W) << 6.  Near cells first make the
// list's k-th distance small early, so later chunks more often hold
// nothing for any lane and skip their merge.
template <int D, int W>
struct NearOrder {
    static constexpr int kSide = 2 * W + 1;
    static constexpr int kCells = D == 3 ? kSide * kSide * kSide : kSide * kSide;
    uint16_t off[kCells];
    constexpr NearOrder() : off{} {
        int k = 0;
        for (int m = 0; m <= D * W * W; ++m) {
            for (int c = 0; c < kCells; ++c) {
                const int dx = c % kSide - W, dy = c / kSide % kSide - W, dz = D == 3 ? c / (kSide * kSide) - W : 0;
                if (dx * dx + dy * dy + dz * dz == m) {
                    off[k++] = static_cast<uint16_t>((dx + W) | (dy + W) << 3 | (dz + W) << 6);
                }
            }
        }
    }
    static constexpr int dx(int o) { return (o & 7) - W; }
    static constexpr int dy(int o) { return (o >> 3 & 7) - W; }
    static constexpr int dz(int o) { return D == 3 ? (o >> 6) - W : 0; }
};

// The cell-block passes' point distance.  Every point and query they take is
// finite (grid_table_kernel disables a cloud holding a non-finite point or
// box; a lane with a non-finite query takes no part), so e = p - q is never
// NaN and point_distance's max(|e|, 0) is |e|; |e|^2 and e^2 are the same
// bits (IEEE products are sign-symmetric, fused or not; an overflowed
// difference squares to inf either way).
template <int D>
__device__ __forceinline__ float point_distance_finite(const float* q, const float4 p) {
    const float pc[3] = {p.x, p.y, p.z};
    float s = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const float e = pc[d] - q[d];
        s = d == 0 ? e * e : __builtin_fmaf(e, e, s);
    }
    return s;
}

// Streams one lane's runs into its list: `runs` is the lane's column of
// packed runs ((first point << 8) | count, kKnnBlock words apart), `nruns`
// of them, `pts` the cloud's accel points.  A chunk takes the rest of the
// current run and the start of the next (one run per chunk measured +13% at
// cfg2, three the same as two; 12 points per chunk slower).
template <int D, int K>
__device__ __forceinline__ void grid_stream(const uint32_t* runs, int nruns, const float4* pts, const float* q,
                                            uint64_t (&best)[K]) {
    constexpr int kChunk = 8;
    // Cursor: run j, its next point s and its end e.
    int j = 0, s = 0, e = 0;
    if (nruns > 0) {
        const uint32_t r = runs[0];
        s = static_cast<int>(r >> 8);
        e = s + static_cast<int>(r & 255u);
    }
    // Moves to the next run with points left, if any.
    const auto advance = [&]() {
        while (s == e && j < nruns - 1) {
            ++j;
            const uint32_t r = runs[j * kKnnBlock];
            s = static_cast<int>(r >> 8);
            e = s + static_cast<int>(r & 255u);
        }
    };
    while (true) {
        advance();
        const int s0 = s;
        const int n0 = min(e - s, kChunk);
        s += n0;
        if (__ballot(n0 > 0) == 0) break;  // every lane's runs are exhausted
        advance();
        const int s1 = s - n0;  // slot u >= n0 takes point s1 + u
        const int n1 = min(e - s, kChunk - n0);
        s += n1;
        float4 p[kChunk];
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const int row = u < n0 ? s0 + u : u < n0 + n1 ? s1 + u : 0;
            p[u] = pts[row];
        }
        uint64_t cand[kChunk];
        uint64_t least = kEmptyKey;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const float dd = point_distance<D>(q, p[u]);
            cand[u] = u < n0 + n1 && dd < kFar ? candidate_key(dd, __float_as_uint(p[u].w)) : kEmptyKey;
            least = key_min(least, cand[u]);
        }
        // A chunk that improves no lane's list needs no merge.
        if (__ballot(least < best[K - 1]) != 0) merge_candidates<K, kChunk>(best, cand);
    }
}

// Distance from the query to the boundary of the block of cells c - w ..
// c + w per axis, where points lie beyond it (a block side at the grid's
// edge has none), less the slack (1e-5 of the larger of the box's extents
// and its coordinates' magnitudes) that covers the rounding of the
// quantisation, of the boundary and of the distances.
template <int D>
__device__ __forceinline__ float grid_safe_margin(const float* q, const float* root, const uint32_t (&c)[D], int shift,
                                                  int G, int w) {
    float margin = INFINITY;
    float size = 0.0f;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        const float lo = root[d], hi = root[D + d];
        const float ext = hi - lo;
        size = fmaxf(size, fmaxf(ext, fmaxf(fabsf(lo), fabsf(hi))));
        const int b0 = static_cast<int>(c[d]) - w, b1 = static_cast<int>(c[d]) + w + 1;
        const float scale = ext / static_cast<float>(1u << grid_axis_bits<D>());
        if (b0 > 0) margin = fminf(margin, q[d] - (lo + static_cast<float>(b0 << shift) * scale));
        if (b1 < G) margin = fminf(margin, (lo + static_cast<float>(b1 << shift) * scale) - q[d]);
    }
    return margin - 1e-5f * size;
}

// Whether the second pass runs (see grid_knn2_kernel).
constexpr bool grid_second_pass(int D, int K) { return D == 3 && (K == 8 || K == 16); }

// A routed search's second structure (the false route's): its node boxes
// (`nr` rows per cloud, row 0 the root box), its level and its clouds'
// first-point tables.  Its clouds' flags follow the first's (flags[B + b]).
struct GridSecond {
    const float* nodes;
    int64_t nr;
    int level;
    const int32_t* table;
};

// One query per lane, in launch order like the traversal (same tile map).
// Failing queries are appended to the failure list (grid_append; bounds[gid]
// their block's k-th distance, FLT_MAX where none was taken).
//
// A lane first reads the runs of its block's cells (first point and count,
// packed into one LDS word per cell: clouds of at most 2^24 points, runs of
// at most 255, more sends the query to the traversal) and then streams
// them as one sequence, kChunk points per merge, a chunk taking the rest of
// one run and the start of the next.  Scanning cell by cell in lockstep,
// a cell cost the wave as many chunks as its fullest lane needed (at 4
// points per cell, nearly always two chunks of 6 somewhere among 64 lanes:
// about 55 merges per wave at cfg2); the stream costs ceil(points / 8) per
// lane.
//
// Routed (kRouted: batched, ordered, spatial output): each lane searches
// the structure its query's route names (locate), with that structure's
// box, level, table and points, its indices offset as in the traversal.
template <int D, int K, bool kOrdered, bool kRouted>
__global__ __launch_bounds__(kKnnBlock) void grid_knn_kernel(KnnArgs a, const float* __restrict__ node_aabbs, int64_t nr,
                                                         int level, const int32_t* __restrict__ table,
                                                         const uint32_t* __restrict__ flags, int32_t* __restrict__ list,
                                                         uint32_t* __restrict__ counts, int64_t seg,
                                                         float* __restrict__ bounds, GridSecond g2) {
    using Order = NearOrder<D, 1>;
    constexpr int kCells = Order::kCells;
    __shared__ uint32_t s_runs[kCells * kKnnBlock];
    const int64_t per_xcd = gridDim.x / kXcds;
    const int64_t tile = (blockIdx.x % kXcds) * per_xcd + blockIdx.x / kXcds;
    if (tile * kKnnBlock >= a.total_q) return;  // surplus tiles (whole waves)
    const int lane = threadIdx.x;
    const int64_t gid = tile * kKnnBlock + lane;
    // Lanes past the last query take no part; a lane whose cloud is
    // disabled goes to the fallback at once (which also handles a corrupt
    // order entry: no result).  A lane on a corrupt entry here takes no part.
    bool valid = gid < a.total_q;
    const int64_t b = valid ? gid / a.M : 0;
    bool ok;
    QueryLoc in{};
    if constexpr (kRouted) {
        // The route names the structure, so the query is located first; the
        // false route's clouds have flags B .. 2B - 1.
        const bool launched = valid;
        if (valid) {
            in = locate<true, false, true, true>(a, gid);
            valid = in.row >= 0;
        }
        ok = valid && flags[(in.second ? a.B : 0) + b] == 0u;
        if (__ballot(ok) == 0) {
            grid_append(list, counts, seg, __ballot(launched), gid);
            if (launched) bounds[gid] = kFar;
            return;
        }
    } else {
        ok = valid && flags[b] == 0u;
        if (__ballot(ok) == 0) {
            grid_append(list, counts, seg, __ballot(valid), gid);
            if (valid) bounds[gid] = kFar;
            return;
        }
        if (valid) {
            in = locate<kOrdered, false, false, true>(a, gid);
            valid = in.row >= 0;
            ok = ok && valid;
        }
    }
    const bool second = kRouted && in.second;
    const int n = kRouted ? in.n : a.num_leaves;
    float q[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        q[d] = valid ? a.queries[in.row * D + d] : 0.0f;
        ok = ok && isfinite(q[d]);
    }
    const float* root = second ? g2.nodes + b * g2.nr * 2 * D : node_aabbs + b * nr * 2 * D;
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        lo[d] = root[d];
        hi[d] = root[D + d];
    }
    const int lv = second ? g2.level : level;
    const int shift = grid_axis_bits<D>() - lv;
    const int G = 1 << lv;
    uint32_t c[D];
    grid_cell<D>(q, lo, hi, shift, c);
    const int64_t cells = int64_t(1) << (D * lv);
    const int32_t* t = (second ? g2.table : table) + b * (cells + 1);
    // The block's runs, nearest cells first.  The search is kept only while
    // the block's point count stays near the cloud's mean (4x); past that,
    // or a run longer than a count field holds, the lane goes to the
    // traversal.
    constexpr Order kOrder{};
    const int cap = 4 * kCells * static_cast<int>((n + cells - 1) / cells);
    int total = 0;
    // Nine cells at a time, every lane loading both table entries of each
    // (a cell outside the grid, or any cell of a lane that is not searching,
    // reads entry 0 and is masked after): the 18 loads then issue together.
    // With each cell's loads under its own branch, every load waited for
    // the one before (54 round trips per wave at 3-D).
    constexpr int kGroup = 9;
    static_assert(kCells % kGroup == 0, "whole groups of cells");
    const bool searching = ok;
    // Per axis, the block's three columns: inside the grid or not, and their
    // Morton bits in the axis's place, so that a cell's id is the OR of its
    // columns' bits (grid_cell_id) and its test two ANDs.  Deriving each
    // cell's id from its coordinates took about 18 instructions per cell,
    // two of them quarter-rate multiplies, under a branch per cell (this
    // pass at cfg2 239.6 -> 228.4 us, 3-D k = 32 258.5 -> 241.6 us, cfg4
    // 556.9 -> 546.5 us).
    uint32_t col_bits[D][3];
    bool col_in[D][3];
#pragma unroll
    for (int d = 0; d < D; ++d) {
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            const int x = static_cast<int>(c[d]) + k - 1;
            col_in[d][k] = x >= 0 && x < G;
            const uint32_t ux = static_cast<uint32_t>(x);
            col_bits[d][k] = (D == 3 ? morton::spread3(ux) : morton::spread2(ux)) << d;
        }
    }
#pragma unroll
    for (int g0 = 0; g0 < kCells; g0 += kGroup) {
        int32_t raw_s[kGroup], raw_e[kGroup];
        bool in[kGroup];
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            const int o = kOrder.off[g0 + u];
            const int kx = Order::dx(o) + 1, ky = Order::dy(o) + 1, kz = D == 3 ? Order::dz(o) + 1 : 1;
            in[u] = searching && col_in[0][kx] && col_in[1][ky] && (D == 2 || col_in[D - 1][kz]);
            const uint32_t id = col_bits[0][kx] | col_bits[1][ky] | (D == 3 ? col_bits[D - 1][kz] : 0u);
            const uint32_t at = in[u] ? id : 0u;
            raw_s[u] = t[at];
            raw_e[u] = t[at + 1];
        }
#pragma unroll
        for (int u = 0; u < kGroup; ++u) {
            // Entries of an enabled cloud lie in [0, n]; clamped all the same.
            const int rs = in[u] ? min(max(raw_s[u], 0), n) : 0;
            const int re = in[u] ? min(max(raw_e[u], rs), n) : 0;
            total += re - rs;
            ok = ok && re - rs <= 255;
            s_runs[(g0 + u) * kKnnBlock + lane] =
                static_cast<uint32_t>(rs) << 8 | static_cast<uint32_t>(min(re - rs, 255));
        }
    }
    ok = ok && total <= cap;
    uint64_t best[K];
#pragma unroll
    for (int i = 0; i < K; ++i) best[i] = candidate_key(kFar, 0xffffffffu);
    // The stream of grid_stream, written out here: as a call it came out at
    // 136 VGPRs instead of 89 at 3-D k = 16 (3 waves per SIMD instead of 5).
    constexpr int kChunk = 8;
    const float4* pts = static_cast<const float4*>(second ? a.accel2 : a.accel) + in.pstart;
    // Cursor: run j, its next point s and its end e (a lane that is not ok
    // starts at the end).
    int j = ok ? 0 : kCells - 1;
    int s = 0, e = 0;
    if (ok) {
        const uint32_t r = s_runs[lane];
        s = static_cast<int>(r >> 8);
        e = s + static_cast<int>(r & 255u);
    }
    // Moves to the next run with points left, if any.
    const auto advance = [&]() {
        while (s == e && j < kCells - 1) {
            ++j;
            const uint32_t r = s_runs[j * kKnnBlock + lane];
            s = static_cast<int>(r >> 8);
            e = s + static_cast<int>(r & 255u);
        }
    };
    // A chunk takes the rest of the current run and the start of the next
    // (one run per chunk measured +13% at cfg2, three the same as two; 12
    // points per chunk slower).
    while (true) {
        advance();
        const int s0 = s;
        const int n0 = min(e - s, kChunk);
        s += n0;
        if (__ballot(n0 > 0) == 0) break;  // every lane's runs are exhausted
        advance();
        const int s1 = s - n0;  // slot u >= n0 takes point s1 + u
        const int n1 = min(e - s, kChunk - n0);
        s += n1;
        // Slot u >= n0 reads row s1 + u >= the next run's start (s1 is it
        // less n0), so every row is non-negative; a slot past n0 + n1 reads
        // at most kChunk - 1 rows past a row the lane was given (rows 0 ..
        // kChunk - 1 for a lane given none), inside the accel buffer, whose
        // record rows follow its point rows, and its key is dropped.
        // Measured against the select form below (padding slots reading row
        // 0), pass 1 at cfg2: 241.7 -> 236.9 us at 3-D k = 16, 261.7 ->
        // 254.6 us at k = 32; but 2-D k = 8 550.7 -> 598.7 us, where padding
        // slots are more common, and 3-D k = 8 takes 82 VGPRs instead of 76
        // (6 -> 5 waves per SIMD).
        float4 p[kChunk];
        if constexpr (D == 3 && K >= 16) {
#pragma unroll
            for (int u = 0; u < kChunk; ++u) p[u] = pts[static_cast<uint32_t>(u < n0 ? s0 + u : s1 + u)];
        } else {
#pragma unroll
            for (int u = 0; u < kChunk; ++u) p[u] = pts[u < n0 ? s0 + u : u < n0 + n1 ? s1 + u : 0];
        }
        uint64_t cand[kChunk];
        uint64_t least = kEmptyKey;
#pragma unroll
        for (int u = 0; u < kChunk; ++u) {
            const float dd = point_distance_finite<D>(q, p[u]);
            cand[u] = u < n0 + n1 && dd < kFar ? candidate_key(dd, __float_as_uint(p[u].w)) : kEmptyKey;
            least = key_min(least, cand[u]);
        }
        // A chunk that improves no lane's list needs no merge.
        if (__ballot(least < best[K - 1]) != 0) merge_candidates<K, kChunk>(best, cand);
    }
    const float safe = grid_safe_margin<D>(q, root, c, shift, G, 1);
    const float worst = __uint_as_float(static_cast<uint32_t>(best[K - 1] >> 32));
    const bool done = ok && safe > 0.0f && worst < safe * safe;
    // Failures with a full list leave it in their result row for the
    // second pass, which goes on from it.
    if (done || (grid_second_pass(D, K) && ok && worst < kFar)) {
        // Derived again rather than held through the scan.
        const QueryLoc out = locate<kOrdered, false, kRouted, true>(a, gid);
        write_results<K, D>(a, out.out_row, best, out.index_offset, out.pstart);
    }
    grid_append(list, counts, seg, __ballot(valid && !done), gid);
    if (valid && !done) bounds[gid] = ok ? worst : kFar;
}

// Second pass over the first pass's failures (list[0 .. *count), launch
// positions; bounds[gid] the k-th distance of the first block's list,
// FLT_MAX where it had none): the block of 5^D cells around the query.  The
// first block's 3^D cells are done: their k nearest points are the list
// the first pass left in the query's result row, which this pass reads
// back.  Of the shell around them it keeps the cells not wholly beyond
// that list's k-th distance (lower bound of their points' distances, short
// by the slack, greater than it: no such point can enter the final list,
// whose k-th distance is at most the bound), streams their points into the
// list, and keeps the result when its k-th distance is inside the block's
// margin, at least two cells.  Failures go to the traversal with the new
// k-th distance, per tile of list positions as in the first pass.
// Run for 3-D k = 8 and 16 only (grid_second_pass).  At cfg2 the first pass
// leaves 13% of the queries, which the traversal answered in 117 us; with
// this pass the whole call measured 0.425 -> 0.386 ms (3-D k = 8: 0.344 ->
// 0.310), but +50% at 3-D k = 4 (0.5 points per cell: 125 cells to cull
// and more first-pass failures), +5% in 2-D (first-pass failures rare: its
// three launches cost more than they save), +4% at k = 32.  Reading the
// first list back instead of scanning the inner block again: this pass
// 81 -> 63 us at cfg2 (the call 0.379 -> 0.378 ms; 3-D k = 8 0.306 ->
// 0.294 ms); it waits on memory more than it computes.
// Routed (kRouted) as in the first pass: each lane takes its route's
// structure, and the list read back has its indices offset.
constexpr int kGridRuns2 = 32;  // kept shell cells per lane (more: the traversal)
template <int D, int K, bool kOrdered, bool kRouted>
__global__ __launch_bounds__(kKnnBlock) void grid_knn2_kernel(KnnArgs a, const float* __restrict__ node_aabbs,
                                                          int64_t nr, int level, const int32_t* __restrict__ table,
                                                          const int32_t* __restrict__ list,
                                                          const uint32_t* __restrict__ counts,
                                                          int32_t* __restrict__ list2, uint32_t* __restrict__ counts2,
                                                          int64_t seg, float* __restrict__ bounds, GridSecond g2) {
    __shared__ uint32_t s_runs[kGridRuns2 * kKnnBlock];
    // A chunk of this work-group's sub-list of the first list (the grid is
    // sized for every query; work-groups past the sub-list's length exit).
    const int64_t listed = counts[grid_sublist() * kCountStride];
    const int64_t at0 = grid_chunk_start();
    if (at0 >= listed) return;  // surplus work-groups (whole waves)
    const int lane = threadIdx.x;
    const bool valid = at0 + lane < listed;
    const int64_t gid = valid ? list[grid_sublist() * seg + at0 + lane] : 0;
    const float seed = valid ? bounds[gid] : kFar;
    // Lanes without a bound (disabled cloud, full block, non-finite query,
    // corrupt order entry) go on to the traversal.
    bool ok = valid && seed < kFar;
    if (__ballot(ok) == 0) {
        grid_append(list2, counts2, seg, __ballot(valid), gid);
        return;
    }
    QueryLoc in{};
    if (ok) {
        in = locate<kOrdered, false, kRouted, true>(a, gid);
        ok = in.row >= 0;
    }
    const bool second = kRouted && in.second;
    const int n = kRouted ? in.n : a.num_leaves;
    const int64_t b = ok ? gid / a.M : 0;
    float q[D];
#pragma unroll
    for (int d = 0; d < D; ++d) q[d] = ok ? a.queries[in.row * D + d] : 0.0f;
    const float* root = second ? g2.nodes + b * g2.nr * 2 * D : node_aabbs + b * nr * 2 * D;
    float lo[D], hi[D];
#pragma unroll
    for (int d = 0; d < D; ++d) {
        lo[d] = root[d];
        hi[d] = root[D + d];
    }
    const int lv = second ? g2.level : level;
    const int shift = grid_axis_bits<D>() - lv;
    const int G = 1 << lv;
    uint32_t c[D];
    grid_cell<D>(q, lo, hi, shift, c);
    // Squared lower bounds of |p_d - q_d| for points in the cells at offset
    // -2 .. 2 on each axis: the distance to the nearer face of the column,
    // short by the slack (as in grid_safe_margin), 0 for the query's own;
    // +inf for a column outside the grid (its cells are never kept).
    float lb[D][5];
    {
        float size = 0.0f;
#pragma unroll
        for (int d = 0; d < D; ++d) size = fmaxf(size, fmaxf(hi[d] - lo[d], fmaxf(fabsf(lo[d]), fabsf(hi[d]))));
        const float slack = 1e-5f * size;
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const float scale = (hi[d] - lo[d]) / static_cast<float>(1u << grid_axis_bits<D>());
            const auto face = [&](int k) { return lo[d] + static_cast<float>((static_cast<int>(c[d]) + k) << shift) * scale; };
            const float f[5] = {q[d] - face(-1), q[d] - face(0), 0.0f, face(1) - q[d], face(2) - q[d]};
#pragma unroll
            for (int k = 0; k < 5; ++k) {
                const float v = fmaxf(f[k] - slack, 0.0f);
                const int x = static_cast<int>(c[d]) + k - 2;
                lb[d][k] = x < 0 || x >= G ? INFINITY : k == 2 ? 0.0f : v * v;
            }
        }
    }
    const int64_t cells = int64_t(1) << (D * lv);
    const int32_t* t = (second ? g2.table : table) + b * (cells + 1);
    // The shell's cells kept, as bits of the 5^D block (bit (ox + 2) + 5 (oy
    // + 2) + 25 (oz + 2) for offset (ox, oy, oz)): those not wholly beyond
    // the bound.  The bits are set without branches and the kept cells then
    // listed bit by bit, a few instructions per cell for the wave where a
    // branch per cell (with its append) cost it about 30 (this pass at cfg2
    // 45.7 -> 38.8 us, at 3-D k = 8 20.7 -> 15.2 us); the cells' order
    // changes no result (the list keeps the k smallest keys of all it is
    // given).  More than kGridRuns2 kept: the traversal.  Then their table
    // entries in batches of 8 whose loads issue together (loading under
    // each cell's own branch, every load waited for the one before).
    constexpr int kSide = 5;
    constexpr int kBlockCells = D == 3 ? kSide * kSide * kSide : kSide * kSide;
    constexpr int kWords = (kBlockCells + 31) / 32;
    uint32_t keep[kWords];
#pragma unroll
    for (int w = 0; w < kWords; ++w) keep[w] = 0u;
#pragma unroll
    for (int i = 0; i < kBlockCells; ++i) {
        const int ox = i % kSide, oy = i / kSide % kSide, oz = D == 3 ? i / (kSide * kSide) : 2;
        // The first block's cells are in the list already.
        if (ox >= 1 && ox <= 3 && oy >= 1 && oy <= 3 && oz >= 1 && oz <= 3) continue;
        float bound = lb[0][ox] + lb[1][oy];
        if constexpr (D == 3) bound += lb[D - 1][oz];
        keep[i / 32] |= (bound > seed ? 0u : 1u) << (i % 32);
    }
    int kept = 0;
#pragma unroll
    for (int w = 0; w < kWords; ++w) kept += __popc(keep[w]);
    ok = ok && kept <= kGridRuns2;
    int nruns = 0;
    if (ok) {
#pragma unroll
        for (int w = 0; w < kWords; ++w) {
            uint32_t m = keep[w];
            while (m != 0u) {
                const int i = w * 32 + __builtin_ctz(m);
                m &= m - 1u;
                uint32_t cell[D];
                cell[0] = static_cast<uint32_t>(static_cast<int>(c[0]) + i % kSide - 2);
                cell[1] = static_cast<uint32_t>(static_cast<int>(c[1]) + i / kSide % kSide - 2);
                if constexpr (D == 3) cell[D - 1] = static_cast<uint32_t>(static_cast<int>(c[D - 1]) + i / (kSide * kSide) - 2);
                s_runs[nruns * kKnnBlock + lane] = grid_cell_id<D>(cell);
                ++nruns;
            }
        }
    }
    if (!ok) nruns = 0;
    constexpr int kBatch = 8;
#pragma unroll
    for (int r0 = 0; r0 < kGridRuns2; r0 += kBatch) {
        if (__ballot(r0 < nruns) == 0) break;
        int32_t raw_s[kBatch], raw_e[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t id = r0 + u < nruns ? s_runs[(r0 + u) * kKnnBlock + lane] : 0u;
            raw_s[u] = t[id];
            raw_e[u] = t[id + 1];
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            if (r0 + u < nruns) {
                // Entries of an enabled cloud lie in [0, n]; clamped all the same.
                const int rs = min(max(raw_s[u], 0), n);
                const int re = min(max(raw_e[u], rs), n);
                ok = ok && re - rs <= 255;
                s_runs[(r0 + u) * kKnnBlock + lane] = static_cast<uint32_t>(rs) << 8 | static_cast<uint32_t>(re - rs);
            }
        }
    }
    // The first block's list, ascending (its k-th distance is the bound),
    // read as 16-byte loads where the outputs allow (wave-uniform tests).
    uint64_t best[K];
    {
        const int64_t* oi = a.out_indices + (ok ? in.out_row : 0) * K;
        const float* od = a.out_distances + (ok ? in.out_row : 0) * K;
        uint32_t ri[K];
        float rd[K];
        if ((reinterpret_cast<uintptr_t>(a.out_indices) & 15u) == 0) {
#pragma unroll
            for (int v = 0; v < K / 2; ++v) {
                const int4 w = reinterpret_cast<const int4*>(oi)[v];
                ri[2 * v] = static_cast<uint32_t>(w.x);
                ri[2 * v + 1] = static_cast<uint32_t>(w.z);
            }
        } else {
#pragma unroll
            for (int i = 0; i < K; ++i) ri[i] = static_cast<uint32_t>(oi[i]);
        }
        if ((reinterpret_cast<uintptr_t>(a.out_distances) & 15u) == 0) {
#pragma unroll
            for (int v = 0; v < K / 4; ++v) {
                const float4 w = reinterpret_cast<const float4*>(od)[v];
                rd[4 * v] = w.x;
                rd[4 * v + 1] = w.y;
                rd[4 * v + 2] = w.z;
                rd[4 * v + 3] = w.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < K; ++i) rd[i] = od[i];
        }
        // A routed list was written with its route's index offset.
        const uint32_t off = static_cast<uint32_t>(in.index_offset);
#pragma unroll
        for (int i = 0; i < K; ++i) best[i] = ok ? candidate_key(rd[i], ri[i] - off) : kEmptyKey;
    }
    grid_stream<D, K>(s_runs + lane, ok ? nruns : 0, static_cast<const float4*>(second ? a.accel2 : a.accel) + in.pstart,
                      q, best);
    const float safe = grid_safe_margin<D>(q, root, c, shift, G, 2);
    const float worst = __uint_as_float(static_cast<uint32_t>(best[K - 1] >> 32));
    const bool done = ok && safe > 0.0f && worst < safe * safe;
    if (done) {
        const QueryLoc out = locate<kOrdered, false, kRouted, true>(a, gid);
        write_results<K, D, true>(a, out.out_row, best, out.index_offset, out.pstart);
    }
    grid_append(list2, counts2, seg, __ballot(valid && !done), gid);
    if (ok && !done) bounds[gid] = worst;
}

template <int D, int K, bool kOrdered, bool kRagged, bool kRouted, bool kAccel, bool kCompact = false>
void launch_one(const KnnArgs& a, unsigned grid, hipStream_t stream) {
    if constexpr (kAccel) knn_accel_kernel<D, K, kOrdered, kRagged, kRouted, kCompact><<<grid, kKnnBlock, 0, stream>>>(a);
    else knn_kernel<D, K, kOrdered, kRagged, kRouted><<<grid, kKnnBlock, 0, stream>>>(a);
}

template <int D, int K, bool kAccel>
hipError_t launch_dk(const KnnArgs& a, bool ragged, hipStream_t stream) {
    // Whole XCD rounds (see knn_query); surplus tiles exit at once.
    const int64_t tiles = (a.total_q + kKnnBlock - 1) / kKnnBlock;
    const unsigned grid = static_cast<unsigned>((tiles + kXcds - 1) / kXcds * kXcds);
    const bool ordered = a.order != nullptr;
    if (a.routes != nullptr) {
        // Routed launches are batched and always ordered (the routed sort).
        if (ragged || !ordered) return hipErrorInvalidValue;
        launch_one<D, K, true, false, true, kAccel>(a, grid, stream);
    } else if constexpr (kAccel && D == 3 && K == 16) {
        // The compact ring (RingStack) where every cloud has at most
        // kCompactCloud points: a ragged call's clouds share its total.
        const bool compact = (ragged ? a.total_points : static_cast<int64_t>(a.num_leaves)) <= kCompactCloud;
        if (compact) {
            if (ragged) {
                if (ordered) launch_one<D, K, true, true, false, true, true>(a, grid, stream);
                else launch_one<D, K, false, true, false, true, true>(a, grid, stream);
            } else {
                if (ordered) launch_one<D, K, true, false, false, true, true>(a, grid, stream);
                else launch_one<D, K, false, false, false, true, true>(a, grid, stream);
            }
        } else if (ragged) {
            if (ordered) launch_one<D, K, true, true, false, true>(a, grid, stream);
            else launch_one<D, K, false, true, false, true>(a, grid, stream);
        } else {
            if (ordered) launch_one<D, K, true, false, false, true>(a, grid, stream);
            else launch_one<D, K, false, false, false, true>(a, grid, stream);
        }
    } else if (ragged) {
        if (ordered) launch_one<D, K, true, true, false, kAccel>(a, grid, stream);
        else launch_one<D, K, false, true, false, kAccel>(a, grid, stream);
    } else {
        if (ordered) launch_one<D, K, true, false, false, kAccel>(a, grid, stream);
        else launch_one<D, K, false, false, false, kAccel>(a, grid, stream);
    }
    return hipGetLastError();
}

template <int D, bool kAccel>
hipError_t launch_d(const KnnArgs& a, int K, bool ragged, hipStream_t stream) {
    switch (K) {
        case 4: return launch_dk<D, 4, kAccel>(a, ragged, stream);
        case 8: return launch_dk<D, 8, kAccel>(a, ragged, stream);
        case 16: return launch_dk<D, 16, kAccel>(a, ragged, stream);
        case 32: return launch_dk<D, 32, kAccel>(a, ragged, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_knn(const KnnArgs& a, int D, int K, bool ragged, hipStream_t stream) {
    if (a.total_q == 0) return hipSuccess;
    return D == 3 ? launch_d<3, false>(a, K, ragged, stream) : launch_d<2, false>(a, K, ragged, stream);
}

hipError_t launch_knn_accel(const KnnArgs& a, int D, int K, bool ragged, hipStream_t stream) {
    if (a.total_q == 0) return hipSuccess;
    return D == 3 ? launch_d<3, true>(a, K, ragged, stream) : launch_d<2, true>(a, K, ragged, stream);
}

// The finest level with at least rho points per cell on average, so that
// the k-th neighbour's distance stays within about one cell (3-D:
// (3k / (4 pi rho))^(1/3) = 0.98 cells at rho = k / 4; 2-D: (k / (pi
// rho))^(1/2) = 0.80 at rho = k / 2), inside the block's one-cell margin
// for most queries (cfg2 87%, cfg4 97% in the CPU model); a level holds
// rho to 2^D rho points per cell.  Measured on uniform 3-D clouds (k-NN
// call, schedule order), the nearest level instead: 2^19 points at k = 16
// gave 2 points per cell and 0.411 ms where 16 per cell take 0.315 (plain
// traversal 0.359); 2^18 at k = 8, 1 per cell and 0.248 ms against 8 per
// cell 0.131 (plain 0.199); 2^20 at k = 4, 0.5 per cell and 0.391 ms
// against 4 per cell 0.271.  k = 32 keeps 4 per cell (0.922 ms at 2^20,
// 32 per cell 1.051, plain 0.954), and so does k = 4 at 2 (1 per cell
// lost at every size measured).  0 when the cloud is too small for a grid
// of at least 4 cells per axis, or where the traversal alone measured
// faster (below); at most 2^24 cells.
int grid_level(int64_t n, int D, int K) {
    // Run starts (at most n) are packed into 24 bits.
    if (n >= (int64_t(1) << 24)) return 0;
    // Where the traversal alone is cheap enough that the block passes'
    // launches and scans do not pay (k-NN call against the traversal,
    // uniform clouds, 2^15 to 2^17 points): k = 4 below 2^17 points per
    // cloud (3-D, +12% to +30%) and in 2-D at every size measured (+9% to
    // +30%; -7% at 2^20); 2-D clouds of 10,000 points (16 of them, k = 8:
    // +24%).
    if (K <= 4 && (D == 2 || n < (int64_t(1) << 17))) return 0;
    if (D == 2 && n < (int64_t(1) << 15)) return 0;
    const double rho = D == 3 ? (K >= 32 ? 4 : std::max(2, K / 4)) : std::max(2, K / 2);
    const double cells = static_cast<double>(n) / rho;
    int l = static_cast<int>(std::floor(std::log2(std::max(cells, 1.0)) / D));
    const int max_l = D == 3 ? 8 : 12;
    if (l < 2) return 0;
    l = std::min(l, max_l);
    // A level that leaves many more points per cell than rho scans too
    // much (16 clouds of 10,000 points at k = 16, 4.9 rho: +17%; of 50,000
    // at k = 8, 6.1 rho: +5%; 4 rho at 2^16 and 2^19 points, k = 16: -17%
    // and -9%).
    if (static_cast<double>(n) / std::ldexp(1.0, D * l) > 4.5 * rho) return 0;
    return l;
}

namespace {
// Workspace: the cells' first-point tables (a routed search's second
// structure's after the first's), the clouds' flags (B, or 2B routed), the
// two failure lists' counts (kGridCounts each, kCountStride words apart),
// the two lists (kGridCounts sub-lists of `seg` entries: the launch
// positions of one XCD share's tiles of one residue mod kGridSubLists), the
// k-th distance bounds.  level2 = 0: not routed.
struct GridLayout {
    size_t table, table2, flags, counts, list, list2, bounds, total;
    int64_t seg;
};
GridLayout grid_layout(int64_t B, int64_t total_q, int level, int D, int level2) {
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    const size_t cells = size_t(1) << (D * level);
    const size_t cells2 = level2 > 0 ? size_t(1) << (D * level2) : 0;
    const int64_t tiles = (total_q + kKnnBlock - 1) / kKnnBlock;
    const int64_t per_xcd = (tiles + kXcds - 1) / kXcds;
    GridLayout g;
    g.seg = (per_xcd + kGridSubLists - 1) / kGridSubLists * kKnnBlock;
    const size_t list_bytes = static_cast<size_t>(kGridCounts * g.seg) * 4;
    g.table = 0;
    g.table2 = up(g.table + static_cast<size_t>(B) * (cells + 1) * 4);
    g.flags = up(g.table2 + (level2 > 0 ? static_cast<size_t>(B) * (cells2 + 1) * 4 : 0));
    g.counts = up(g.flags + static_cast<size_t>(B) * (level2 > 0 ? 2 : 1) * 4);
    g.list = up(g.counts + static_cast<size_t>(2 * kGridCounts * kCountStride) * 4);
    g.list2 = up(g.list + list_bytes);
    g.bounds = up(g.list2 + list_bytes);
    g.total = up(g.bounds + static_cast<size_t>(total_q) * 4);
    return g;
}

// Pass 1 (pass == 1: failures to `list`) or pass 2 (over `list`, failures
// to `list2`).  Routed launches are ordered (the routed sort).
template <int D, int K>
void launch_grid_dk(const KnnArgs& a, int pass, const float* node_aabbs, int64_t nr, int level, int32_t* table,
                    uint32_t* flags, int32_t* list, uint32_t* counts, int32_t* list2, uint32_t* counts2, int64_t seg,
                    float* bounds, const GridSecond& g2, hipStream_t stream) {
    const int64_t tiles = (a.total_q + kKnnBlock - 1) / kKnnBlock;
    const unsigned grid = static_cast<unsigned>((tiles + kXcds - 1) / kXcds * kXcds);
    const bool ordered = a.order != nullptr;
    const bool routed = a.routes != nullptr;
    if (pass == 1) {
        if (routed) {
            grid_knn_kernel<D, K, true, true><<<grid, kKnnBlock, 0, stream>>>(a, node_aabbs, nr, level, table, flags,
                                                                             list, counts, seg, bounds, g2);
        } else if (ordered) {
            grid_knn_kernel<D, K, true, false><<<grid, kKnnBlock, 0, stream>>>(a, node_aabbs, nr, level, table, flags,
                                                                              list, counts, seg, bounds, g2);
        } else {
            grid_knn_kernel<D, K, false, false><<<grid, kKnnBlock, 0, stream>>>(a, node_aabbs, nr, level, table, flags,
                                                                               list, counts, seg, bounds, g2);
        }
    } else if (routed) {
        grid_knn2_kernel<D, K, true, true><<<grid, kKnnBlock, 0, stream>>>(a, node_aabbs, nr, level, table, list,
                                                                          counts, list2, counts2, seg, bounds, g2);
    } else if (ordered) {
        grid_knn2_kernel<D, K, true, false><<<grid, kKnnBlock, 0, stream>>>(a, node_aabbs, nr, level, table, list,
                                                                           counts, list2, counts2, seg, bounds, g2);
    } else {
        grid_knn2_kernel<D, K, false, false><<<grid, kKnnBlock, 0, stream>>>(a, node_aabbs, nr, level, table, list,
                                                                            counts, list2, counts2, seg, bounds, g2);
    }
}

template <int D>
void launch_grid_table(const KnnArgs& a, const void* accel, int n, const float* node_aabbs, int64_t nr, int level,
                       int32_t* table, uint32_t* flags, hipStream_t stream) {
    const int64_t pts = a.B * static_cast<int64_t>(n);
    const unsigned tgrid = static_cast<unsigned>((pts + kBlock - 1) / kBlock);
    grid_table_kernel<D><<<tgrid, kBlock, 0, stream>>>(static_cast<const float4*>(accel), node_aabbs, nr, a.B, n,
                                                       level, table, flags);
}
}  // namespace

size_t grid_workspace_bytes(int64_t B, int64_t total_q, int level, int D, int level2) {
    return grid_layout(B, total_q, level, D, level2).total;
}

hipError_t launch_grid_knn(const KnnArgs& args, const float* node_aabbs, int64_t nr, int level, int D, int K,
                           void* ws, hipStream_t stream, const float* node_aabbs2, int64_t nr2, int level2) {
    if (args.total_q == 0) return hipSuccess;
    if (level < 2 || args.total_q >= (int64_t(1) << 31) || args.M <= 0) return hipErrorInvalidValue;
    const bool routed = args.routes != nullptr;
    // A routed search is ordered with spatial output (the routed binding's)
    // and has both structures' grids; a plain one has no second structure.
    if (routed && (args.order == nullptr || !args.spatial_output || args.out_positions != nullptr ||
                   level2 < 2 || node_aabbs2 == nullptr || args.accel2 == nullptr)) {
        return hipErrorInvalidValue;
    }
    if (!routed && level2 != 0) return hipErrorInvalidValue;
    const GridLayout g = grid_layout(args.B, args.total_q, level, D, level2);
    char* base = static_cast<char*>(ws);
    int32_t* table = reinterpret_cast<int32_t*>(base + g.table);
    uint32_t* flags = reinterpret_cast<uint32_t*>(base + g.flags);
    uint32_t* counts = reinterpret_cast<uint32_t*>(base + g.counts);
    uint32_t* counts2 = counts + kGridCounts * kCountStride;
    int32_t* list = reinterpret_cast<int32_t*>(base + g.list);
    int32_t* list2 = reinterpret_cast<int32_t*>(base + g.list2);
    float* bounds = reinterpret_cast<float*>(base + g.bounds);
    const GridSecond g2{node_aabbs2, nr2, level2, reinterpret_cast<const int32_t*>(base + g.table2)};
    const int64_t nflags = args.B * (routed ? 2 : 1);
    const int64_t init = std::max<int64_t>(nflags, 2 * kGridCounts);
    grid_init_kernel<<<static_cast<unsigned>((init + kBlock - 1) / kBlock), kBlock, 0, stream>>>(flags, nflags, counts,
                                                                                                2 * kGridCounts);
    auto tables = [&](auto tab) {
        tab(args, args.accel, args.num_leaves, node_aabbs, nr, level, table, flags, stream);
        if (routed) {
            tab(args, args.accel2, args.num_leaves2, node_aabbs2, nr2, level2,
                reinterpret_cast<int32_t*>(base + g.table2), flags + args.B, stream);
        }
    };
    if (D == 3) tables(launch_grid_table<3>);
    else tables(launch_grid_table<2>);
    const int passes = grid_second_pass(D, K) ? 2 : 1;
    for (int pass = 1; pass <= passes; ++pass) {
        auto run = [&](auto dk) {
            dk(args, pass, node_aabbs, nr, level, table, flags, list, counts, list2, counts2, g.seg, bounds, g2,
               stream);
        };
        // k in {4, 8, 16, 32} (supported_k).
        if (D == 3) {
            switch (K) {
                case 4: run(launch_grid_dk<3, 4>); break;
                case 8: run(launch_grid_dk<3, 8>); break;
                case 16: run(launch_grid_dk<3, 16>); break;
                case 32: run(launch_grid_dk<3, 32>); break;
                default: return hipErrorInvalidValue;
            }
        } else {
            switch (K) {
                case 4: run(launch_grid_dk<2, 4>); break;
                case 8: run(launch_grid_dk<2, 8>); break;
                case 16: run(launch_grid_dk<2, 16>); break;
                case 32: run(launch_grid_dk<2, 32>); break;
                default: return hipErrorInvalidValue;
            }
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // The fallback: the accel traversal over the last list (its grid sized
    // for every query; work-groups past their segment's length exit at
    // once), routed where the search is.
    KnnArgs f = args;
    f.fb_list = passes == 2 ? list2 : list;
    f.fb_bound = bounds;
    f.fb_count = passes == 2 ? counts2 : counts;
    f.fb_seg = g.seg;
    return launch_knn_accel(f, D, K, false, stream);
}

}  // namespace tbvh
