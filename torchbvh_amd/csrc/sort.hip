// Segmented stable LSD radix sort of (u32 key, u32 local index) pairs.
//
// Replaces the reference's `cub::DeviceSegmentedRadixSort::SortPairs` calls
// (torchbvh/csrc/bvh_build.cu:580-594, morton_sort.cu:242-256).  The contract
// that matters for parity: within each segment the output is ordered by key,
// and equal keys keep ascending original (local) index — LSD passes of a
// stable counting sort give exactly that.
//
// Design (gfx950): 8-bit digits, kSortTile = 4096 keys per tile, 256-thread
// work-groups, tiles never straddle segments.  The Morton kernel accumulates
// every pass's per-segment digit histogram, so each pass is one kernel
// ("onesweep": Adinets & Merrill, 2022):
//   1. the work-group takes the next tile ticket (tickets follow dispatch
//      order, so every lower ticket belongs to a running or finished group);
//   2. ranks its keys stably (wave64 ballot matching, striped order);
//   3. publishes each digit's count, then looks back over earlier tiles of
//      its segment, summing published counts until it meets an inclusive
//      prefix, and publishes its own inclusive prefix;
//   4. stages the tile in LDS in digit order and writes each digit run
//      contiguously at segment start + digit start + prefix.
// Status words pack flag and count in one 32-bit word and are read and
// written with agent-scope atomics, so they are coherent across XCDs.  A
// group publishes all its aggregates before it waits on anyone, so every
// wait ends; the spin is also bounded and a shared abort flag ends all spins
// at once should that bound ever be reached (the output is then invalid, but
// the kernel exits).
#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

// Work-group size of a sort pass: 8 waves share a 4096-key tile, so each
// wave ranks 512 keys (measured on MI355X: ~10% faster per pass than 4
// waves, no gain from 16).
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kItems = kSortTile / kThreads;  // keys per thread
static_assert(kThreads >= kRadix && kSortTile % kThreads == 0, "sort tiling");
constexpr uint32_t kFlagAggregate = 1u << 30;
constexpr uint32_t kFlagPrefix = 2u << 30;
constexpr uint32_t kCountMask = (1u << 30) - 1;
constexpr int kSpinLimit = 1 << 20;

__device__ __forceinline__ uint32_t load_status(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_status(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

template <bool kFirst, bool kLast>
__global__ __launch_bounds__(kThreads) void onesweep_kernel(const Segment* __restrict__ segs, int S,
                                                            int64_t tiles_total, SortPass pass) {
    __shared__ int64_t s_tile;
    __shared__ int s_seg;
    __shared__ uint32_t s_keys[kSortTile];
    __shared__ uint32_t s_vals[kSortTile];
    __shared__ uint32_t s_cnt[kWaves][kRadix];
    __shared__ uint32_t s_start[kRadix];
    __shared__ uint32_t s_base[kRadix];
    __shared__ uint32_t s_scan[kWaves];
    if (threadIdx.x == 0) {
        const int64_t t = atomicAdd(pass.ticket, 1u);
        s_tile = t;
        s_seg = t < tiles_total
                    ? find_segment([&](int i) { return static_cast<int64_t>(segs[i].tile_first); }, S, t)
                    : 0;
    }
    for (int i = threadIdx.x; i < kWaves * kRadix; i += kThreads) (&s_cnt[0][0])[i] = 0u;
    __syncthreads();
    const int64_t t = s_tile;
    if (t >= tiles_total) return;
    const Segment g = segs[s_seg];
    const int lt = static_cast<int>(t - g.tile_first);
    uint32_t* status = pass.status + t * kRadix;
    if (lt >= g.tiles) {
        // A ticket past the segment's last tile (surplus grid): nothing to
        // sort, but publish zero prefixes so no later tile can wait on it.
        if (threadIdx.x < kRadix) store_status(status + threadIdx.x, kFlagPrefix);
        return;
    }
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);
    const int shift = pass.shift;

    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t key[kItems], val[kItems], rank[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int pos = wave * kWave * kItems + i * kWave + lane;
        const bool valid = pos < count;
        key[i] = valid ? pass.keys_in[row0 + pos] : 0xffffffffu;
        if constexpr (kFirst) {
            val[i] = static_cast<uint32_t>(lt * kSortTile + pos);
        } else {
            val[i] = valid ? pass.vals_in[row0 + pos] : 0u;
        }
    }
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int pos = wave * kWave * kItems + i * kWave + lane;
        const bool valid = pos < count;
        const uint32_t digit = (key[i] >> shift) & (kRadix - 1);
        const uint64_t peers = match_digit(digit, valid);
        const uint32_t before = static_cast<uint32_t>(__popcll(peers & below));
        const uint32_t prior = valid ? s_cnt[wave][digit] : 0u;
        __builtin_amdgcn_wave_barrier();
        if (valid && before == 0) s_cnt[wave][digit] = prior + static_cast<uint32_t>(__popcll(peers));
        __builtin_amdgcn_wave_barrier();
        rank[i] = prior + before;
    }
    __syncthreads();

    // Thread d < kRadix owns digit d: tile count, publish, look back.
    const int d = threadIdx.x;
    uint32_t tile_count = 0, before_tiles = 0, seg_count = 0;
    if (d < kRadix) {
        uint32_t run = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = s_cnt[w][d];
            s_cnt[w][d] = run;
            run += c;
        }
        tile_count = run;
        if (lt == 0) {
            store_status(status + d, kFlagPrefix | tile_count);
        } else {
            store_status(status + d, kFlagAggregate | tile_count);
            for (int64_t j = t - 1;; --j) {
                const uint32_t* other = pass.status + j * kRadix + d;
                uint32_t v = load_status(other);
                int spins = 0;
                while ((v >> 30) == 0) {
                    if (++spins > kSpinLimit) {
                        store_status(pass.abort, 1u);
                    }
                    if ((spins & 63) == 0 && load_status(pass.abort) != 0u) {
                        v = kFlagPrefix;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    v = load_status(other);
                }
                before_tiles += v & kCountMask;
                if ((v & ~kCountMask) == kFlagPrefix) break;
            }
            store_status(status + d, kFlagPrefix | ((before_tiles + tile_count) & kCountMask));
        }
        seg_count = pass.hist[static_cast<int64_t>(s_seg) * kRadix + d];
    }
    // Digit starts of the segment from its global histogram; tile-local
    // digit starts from the tile counts (threads >= kRadix add zeros).
    const uint32_t digit_start = block_exclusive_sum<kThreads>(seg_count, s_scan);
    const uint32_t local_start = block_exclusive_sum<kThreads>(tile_count, s_scan);
    if (d < kRadix) {
        s_base[d] = digit_start + before_tiles;
        s_start[d] = local_start;
    }
    __syncthreads();

#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int pos = wave * kWave * kItems + i * kWave + lane;
        if (pos < count) {
            const uint32_t digit = (key[i] >> shift) & (kRadix - 1);
            const uint32_t at = min(s_start[digit] + s_cnt[wave][digit] + rank[i],
                                    static_cast<uint32_t>(kSortTile - 1));
            s_keys[at] = key[i];
            s_vals[at] = val[i];
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < count; j += kThreads) {
        const uint32_t k = s_keys[j];
        const uint32_t digit = (k >> shift) & (kRadix - 1);
        const uint32_t rel = s_base[digit] + (j - s_start[digit]);
        if (rel >= static_cast<uint32_t>(g.n)) continue;  // unreachable when counts agree
        const int64_t row = g.start + rel;
        if constexpr (kLast) {
            pass.idx_out[row] = static_cast<int64_t>(s_vals[j]);
            if (pass.keys_out) pass.keys_out[row] = k;
        } else {
            pass.keys_out[row] = k;
            pass.vals_out[row] = s_vals[j];
        }
    }
}

}  // namespace

hipError_t launch_sort(const Segment* segs, int64_t S, int64_t tiles, SortBits bits,
                       const SortBuffers& b, int64_t* order, uint32_t* sorted_keys,
                       hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(tiles);
    const int passes = bits.passes();
    const int Si = static_cast<int>(S);
    uint32_t* kin = b.keys_a;
    uint32_t* vin = b.vals_a;
    uint32_t* kout = b.keys_b;
    uint32_t* vout = b.vals_b;
    for (int p = 0; p < passes; ++p) {
        SortPass pass;
        pass.keys_in = kin;
        pass.vals_in = vin;
        pass.keys_out = kout;
        pass.vals_out = vout;
        pass.idx_out = order;
        pass.hist = b.hist + static_cast<int64_t>(p) * S * kRadix;
        pass.status = b.status + static_cast<int64_t>(p) * tiles * kRadix;
        pass.ticket = b.tickets + p;
        pass.abort = b.tickets + kMaxSortPasses;
        pass.shift = bits.first_bit + p * kRadixBits;
        const bool first = p == 0;
        const bool last = p == passes - 1;
        if (last) pass.keys_out = sorted_keys;
        if (first && last) {
            onesweep_kernel<true, true><<<grid, kThreads, 0, stream>>>(segs, Si, tiles, pass);
        } else if (first) {
            onesweep_kernel<true, false><<<grid, kThreads, 0, stream>>>(segs, Si, tiles, pass);
        } else if (last) {
            onesweep_kernel<false, true><<<grid, kThreads, 0, stream>>>(segs, Si, tiles, pass);
        } else {
            onesweep_kernel<false, false><<<grid, kThreads, 0, stream>>>(segs, Si, tiles, pass);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        uint32_t* tk = kin; kin = kout; kout = tk;
        uint32_t* tv = vin; vin = vout; vout = tv;
    }
    return hipSuccess;
}

}  // namespace tbvh
