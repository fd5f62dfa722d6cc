// Segmented stable LSD radix sort of (u32 key, u32 local index) pairs.
//
// Replaces the reference's `cub::DeviceSegmentedRadixSort::SortPairs` calls
// (torchbvh/csrc/bvh_build.cu:580-594, morton_sort.cu:242-256).  The contract
// that matters for parity: within each segment the output is ordered by key,
// and equal keys keep ascending original (local) index — LSD passes of a
// stable counting sort give exactly that.
//
// Design (gfx950): 8-bit digits, kSortTile = 4096 keys per tile, 256-thread
// work-groups, tiles never straddle segments.  Per pass:
//   upsweep  per-tile digit counts (wave64 ballot matching, no atomics)
//   spine    one wave per (segment, digit): scatter base of every tile
//   scatter  rank keys inside the tile (stable), stage the tile in LDS in
//            digit order, then write each digit run contiguously
// The digit-0 counts come from the Morton kernel, so pass 0 has no upsweep;
// pass 0 synthesises the values (local row index) and the last pass writes
// the int64 indices directly.
#include "tbvh_internal.hpp"

namespace tbvh {
namespace {

constexpr int kWaves = kBlock / kWave;
constexpr int kItems = kSortTile / kBlock;

__device__ __forceinline__ int tile_segment(const Segment* segs, int S, int64_t t, int* s_seg) {
    if (threadIdx.x == 0) {
        *s_seg = find_segment([&](int i) { return static_cast<int64_t>(segs[i].tile_first); }, S, t);
    }
    __syncthreads();
    return *s_seg;
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

__global__ __launch_bounds__(kBlock) void upsweep_kernel(const Segment* __restrict__ segs, int S,
                                                         const uint32_t* __restrict__ keys, int shift,
                                                         uint32_t* __restrict__ hist,
                                                         uint32_t* __restrict__ dpre) {
    __shared__ int s_seg;
    __shared__ uint32_t s_cnt[kWaves][kRadix];
    __shared__ uint32_t s_scan[kWaves];
    const int64_t t = blockIdx.x;
    const Segment g = segs[tile_segment(segs, S, t, &s_seg)];
    const int lt = static_cast<int>(t - g.tile_first);
    if (lt >= g.tiles) return;
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);
    for (int i = threadIdx.x; i < kWaves * kRadix; i += kBlock) (&s_cnt[0][0])[i] = 0u;
    __syncthreads();
    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll 4
    for (int i = 0; i < kItems; ++i) {
        const int pos = wave * kWave * kItems + i * kWave + lane;
        const bool valid = pos < count;
        const uint32_t key = valid ? keys[row0 + pos] : 0u;
        const uint32_t digit = (key >> shift) & (kRadix - 1);
        const uint64_t peers = match_digit(digit, valid);
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

// One wave per (segment, digit).  Input, per segment block laid out
// digit-major ([digit][tile]): hist = tile counts, dpre = per-tile count of
// smaller digits.  Output (in place over hist): the row, relative to the
// segment start, at which the tile's run of this digit starts =
//   #(keys of the segment with a smaller digit)
//   + #(keys with this digit in earlier tiles of the segment).
__global__ __launch_bounds__(kBlock) void spine_kernel(const Segment* __restrict__ segs, int S,
                                                       uint32_t* __restrict__ hist,
                                                       const uint32_t* __restrict__ dpre) {
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * kWaves + threadIdx.x / kWave;
    const int64_t s = gw / kRadix;
    if (s >= S) return;
    const int d = static_cast<int>(gw % kRadix);
    const Segment g = segs[s];
    const int lane = lane_id();
    const int64_t blk = static_cast<int64_t>(kRadix) * g.tile_first + static_cast<int64_t>(d) * g.tiles;
    uint32_t smaller = 0;
    for (int j = lane; j < g.tiles; j += kWave) smaller += dpre[blk + j];
    smaller = wave_sum(smaller);
    // Rows are < 2^31, so the digit base fits 32 bits relative to the segment.
    uint32_t carry = smaller;
    for (int j0 = 0; j0 < g.tiles; j0 += kWave) {
        const int j = j0 + lane;
        const uint32_t c = j < g.tiles ? hist[blk + j] : 0u;
        const uint32_t incl = wave_inclusive_sum(c);
        if (j < g.tiles) hist[blk + j] = carry + incl - c;
        carry += __shfl(incl, kWave - 1, kWave);
    }
}

// base[] rows are relative to the segment start (segments hold < 2^31 rows).
template <bool kFirst, bool kLast>
__global__ __launch_bounds__(kBlock) void scatter_kernel(const Segment* __restrict__ segs, int S,
                                                         const uint32_t* __restrict__ keys_in,
                                                         const uint32_t* __restrict__ vals_in,
                                                         uint32_t* __restrict__ keys_out,
                                                         uint32_t* __restrict__ vals_out,
                                                         int64_t* __restrict__ idx_out,
                                                         const uint32_t* __restrict__ base, int shift) {
    __shared__ int s_seg;
    __shared__ uint32_t s_keys[kSortTile];
    __shared__ uint32_t s_vals[kSortTile];
    __shared__ uint32_t s_cnt[kWaves][kRadix];
    __shared__ uint32_t s_start[kRadix];
    __shared__ uint32_t s_base[kRadix];
    __shared__ uint32_t s_scan[kWaves];
    const int64_t t = blockIdx.x;
    const Segment g = segs[tile_segment(segs, S, t, &s_seg)];
    const int lt = static_cast<int>(t - g.tile_first);
    if (lt >= g.tiles) return;
    const int64_t row0 = g.start + static_cast<int64_t>(lt) * kSortTile;
    const int count = min(kSortTile, g.n - lt * kSortTile);
    for (int i = threadIdx.x; i < kWaves * kRadix; i += kBlock) (&s_cnt[0][0])[i] = 0u;
    s_base[threadIdx.x] = base[static_cast<int64_t>(kRadix) * g.tile_first +
                               static_cast<int64_t>(threadIdx.x) * g.tiles + lt];
    __syncthreads();

    const int lane = lane_id();
    const int wave = threadIdx.x / kWave;
    const uint64_t below = (1ull << lane) - 1ull;
    uint32_t key[kItems], val[kItems], rank[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int pos = wave * kWave * kItems + i * kWave + lane;
        const bool valid = pos < count;
        key[i] = valid ? keys_in[row0 + pos] : 0xffffffffu;
        if constexpr (kFirst) {
            val[i] = static_cast<uint32_t>(lt * kSortTile + pos);
        } else {
            val[i] = valid ? vals_in[row0 + pos] : 0u;
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
    {
        const int d = threadIdx.x;
        uint32_t run = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = s_cnt[w][d];
            s_cnt[w][d] = run;
            run += c;
        }
        s_start[d] = block_exclusive_sum(run, s_scan);
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
    for (int j = threadIdx.x; j < count; j += kBlock) {
        const uint32_t k = s_keys[j];
        const uint32_t digit = (k >> shift) & (kRadix - 1);
        const uint32_t rel = s_base[digit] + (j - s_start[digit]);
        if (rel >= static_cast<uint32_t>(g.n)) continue;  // unreachable when counts agree
        const int64_t row = g.start + rel;
        if constexpr (kLast) {
            idx_out[row] = static_cast<int64_t>(s_vals[j]);
        } else {
            keys_out[row] = k;
            vals_out[row] = s_vals[j];
        }
    }
}

}  // namespace

hipError_t launch_sort(const Segment* segs, int64_t S, int64_t tiles, int key_bits,
                       const SortBuffers& b, int64_t* order, hipStream_t stream) {
    const unsigned grid = static_cast<unsigned>(tiles);
    const unsigned spine_grid = static_cast<unsigned>((S * kRadix + kWaves - 1) / kWaves);
    const int passes = (key_bits + kRadixBits - 1) / kRadixBits;
    const int Si = static_cast<int>(S);
    uint32_t* kin = b.keys_a;
    uint32_t* vin = b.vals_a;
    uint32_t* kout = b.keys_b;
    uint32_t* vout = b.vals_b;
    for (int p = 0; p < passes; ++p) {
        const int shift = p * kRadixBits;
        if (p > 0) upsweep_kernel<<<grid, kBlock, 0, stream>>>(segs, Si, kin, shift, b.hist, b.dpre);
        spine_kernel<<<spine_grid, kBlock, 0, stream>>>(segs, Si, b.hist, b.dpre);
        const bool first = p == 0;
        const bool last = p == passes - 1;
        if (first && last) {
            scatter_kernel<true, true><<<grid, kBlock, 0, stream>>>(segs, Si, kin, vin, kout, vout, order, b.hist, shift);
        } else if (first) {
            scatter_kernel<true, false><<<grid, kBlock, 0, stream>>>(segs, Si, kin, vin, kout, vout, order, b.hist, shift);
        } else if (last) {
            scatter_kernel<false, true><<<grid, kBlock, 0, stream>>>(segs, Si, kin, vin, kout, vout, order, b.hist, shift);
        } else {
            scatter_kernel<false, false><<<grid, kBlock, 0, stream>>>(segs, Si, kin, vin, kout, vout, order, b.hist, shift);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        uint32_t* tk = kin; kin = kout; kout = tk;
        uint32_t* tv = vin; vin = vout; vout = tv;
    }
    return hipSuccess;
}

}  // namespace tbvh
