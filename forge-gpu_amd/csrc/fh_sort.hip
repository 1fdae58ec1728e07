// fh_sort.hip -- stable LSD radix sort of (key, value) pairs for gfx950.
//
// Replaces RadixSorter::sort (forge-runtime/src/radix_sort.rs:79-220), whose 4-bit passes
// re-read every earlier block's histogram per block and every earlier key per key.  Design:
//   k_begin        bump the look-back epoch, clear the digit histograms and tile counters
//   k_hist_keys /  one read of the keys builds the 256-bin histograms of ALL 8-bit passes
//   k_hash_hist    (k_hash_hist computes the keys from positions on the fly: the hash of
//                  HashGrid::build, hashgrid.rs:89-92, fused with the histogram)
//   k_onesweep     one kernel per 8-bit pass: a 4096-key tile per workgroup, ranked with
//                  64-lane ballot match-any, digit offsets from a decoupled look-back over
//                  dynamically numbered tiles, then staged in LDS in digit order so the
//                  global scatter writes contiguous runs.
// Stability: within a tile the rank of a key counts the equal digits before it in input order
// (earlier items, earlier lanes, earlier waves); across tiles the look-back prefix counts the
// equal digits of all earlier tiles.  Equal keys therefore keep their input order, which is
// the `sort_by_key` contract of tests/radix_sort_test.rs:111-127.
#include "fh_internal.hpp"

namespace fh {

// ---------------------------------------------------------------------------------------------
__global__ void k_begin(Control* ctl) {
    const int t = threadIdx.x;
    for (int i = t; i < kMaxPasses * 256; i += blockDim.x) (&ctl->hist[0][0])[i] = 0u;
    if (t == 0) {
        uint32_t e = (ctl->epoch + 1u) & kEpochMask;
        ctl->epoch = e ? e : 1u;
        for (int p = 0; p < kMaxPasses; p++) ctl->tile_ctr[p] = 0u;
        ctl->scan_ctr = 0u;
        ctl->heavy_count = 0u;
    }
}

hipError_t launch_begin(fh_ctx* c) {
    tbeg(c, KID_BEGIN);
    k_begin<<<1, 256, 0, c->stream>>>(c->ctl);
    tend(c, KID_BEGIN);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Add one digit per lane to a per-wave LDS histogram.  When the whole wave holds the same digit
// (skewed top digits: c1's top byte is always 0) one lane adds the population instead of 64
// conflicting LDS atomics.
__device__ __forceinline__ void wave_hist_add(uint32_t* h, uint32_t d, bool valid) {
    uint64_t act = __ballot(valid);
    if (act == 0) return;
    uint32_t d0 = __shfl(d, __ffsll((unsigned long long)act) - 1, kWave);
    bool same = __all(!valid || d == d0);
    if (same) {
        if ((threadIdx.x & 63) == __ffsll((unsigned long long)act) - 1)
            atomicAdd(&h[d0], (uint32_t)__popcll(act));
    } else if (valid) {
        atomicAdd(&h[d], 1u);
    }
}

// Shared tail of the histogram kernels: reduce the 4 per-wave histograms and add the nonzero
// bins to the global ones.
__device__ __forceinline__ void flush_hist(uint32_t (*sh)[kMaxPasses][256], Control* ctl,
                                           uint32_t passes) {
    __syncthreads();
    for (uint32_t p = 0; p < passes; p++) {
        uint32_t d = threadIdx.x;  // 256 threads, one bin each
        uint32_t s = sh[0][p][d] + sh[1][p][d] + sh[2][p][d] + sh[3][p][d];
        if (s) atomicAdd(&ctl->hist[p][d], s);
    }
}

__global__ __launch_bounds__(256) void k_hist_keys(const uint32_t* __restrict__ keys, uint32_t n,
                                                   uint32_t num_bits, Control* ctl) {
    __shared__ uint32_t sh[4][kMaxPasses][256];
    const int wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * kMaxPasses * 256; i += 256) (&sh[0][0][0])[i] = 0u;
    __syncthreads();
    const uint32_t passes = passes_for_bits(num_bits);
    const uint32_t stride = gridDim.x * 256u;
    // Trip count is uniform across the block (it depends only on the loop base).
    for (uint32_t base = blockIdx.x * 256u; base < n; base += stride) {
        uint32_t i = base + threadIdx.x;
        bool valid = i < n;
        uint32_t k = valid ? keys[i] : 0u;
        for (uint32_t p = 0; p < passes; p++) {
            uint32_t bits = min(8u, num_bits - 8u * p);
            uint32_t d = (k >> (8u * p)) & ((1u << bits) - 1u);
            wave_hist_add(sh[wave][p], d, valid);
        }
    }
    flush_hist(sh, ctl, passes);
}

hipError_t launch_hist_keys(fh_ctx* c, const uint32_t* keys, uint32_t n, uint32_t num_bits) {
    uint32_t blocks = ceil_div(n, 256u * 16u);
    if (blocks < 1) blocks = 1;
    if (blocks > 2048) blocks = 2048;
    tbeg(c, KID_HIST);
    k_hist_keys<<<blocks, 256, 0, c->stream>>>(keys, n, num_bits, c->ctl);
    tend(c, KID_HIST);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_hash_hist(const float* __restrict__ x,
                                                   const float* __restrict__ y,
                                                   const float* __restrict__ z, uint32_t stride,
                                                   uint32_t n, GridDesc g, uint32_t num_bits,
                                                   uint32_t* __restrict__ keys_out,
                                                   uint32_t* __restrict__ vals_out,
                                                   Control* ctl) {
    __shared__ uint32_t sh[4][kMaxPasses][256];
    const int wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * kMaxPasses * 256; i += 256) (&sh[0][0][0])[i] = 0u;
    __syncthreads();
    const uint32_t passes = passes_for_bits(num_bits);
    const uint32_t gstride = gridDim.x * 256u;
    for (uint32_t base = blockIdx.x * 256u; base < n; base += gstride) {
        uint32_t i = base + threadIdx.x;
        bool valid = i < n;
        uint32_t k = 0;
        if (valid) {
            size_t o = (size_t)i * stride;
            k = cell_of(x[o], y[o], z[o], g);
            if (keys_out) keys_out[i] = k;
            if (vals_out) vals_out[i] = i;
        }
        for (uint32_t p = 0; p < passes; p++) {
            uint32_t bits = min(8u, num_bits - 8u * p);
            uint32_t d = (k >> (8u * p)) & ((1u << bits) - 1u);
            wave_hist_add(sh[wave][p], d, valid);
        }
    }
    flush_hist(sh, ctl, passes);
}

hipError_t launch_hash_hist(fh_ctx* c, const float* x, const float* y, const float* z,
                            uint32_t stride, uint32_t n, const GridDesc& g, uint32_t num_bits,
                            uint32_t* keys_out, uint32_t* vals_out) {
    uint32_t blocks = ceil_div(n, 256u * 8u);
    if (blocks < 1) blocks = 1;
    if (blocks > 2048) blocks = 2048;
    tbeg(c, KID_HASH);
    k_hash_hist<<<blocks, 256, 0, c->stream>>>(x, y, z, stride, n, g, num_bits, keys_out,
                                               vals_out, c->ctl);
    tend(c, KID_HASH);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// One 8-bit (or narrower, for the last pass) digit pass.
__global__ __launch_bounds__(kSortThreads) void k_onesweep(
    const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, Control* ctl, uint32_t pass,
    uint64_t* __restrict__ lookback, uint32_t n, uint32_t shift, uint32_t pbits) {
    __shared__ uint32_t s_keys[kSortTile];
    __shared__ uint32_t s_vals[kSortTile];
    __shared__ uint32_t s_wcnt[4][256];  // per-wave digit counts, then per-wave digit offsets
    __shared__ uint32_t s_dstart[256];   // first slot of digit d in the tile's digit order
    __shared__ uint32_t s_gbase[256];    // global index of slot 0 of digit d's run, minus s_dstart
    __shared__ uint32_t s_scan[4];
    __shared__ uint32_t s_tile;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t mask = (1u << pbits) - 1u;
    if (tid == 0) s_tile = atomicAdd(&ctl->tile_ctr[pass], 1u);
    for (int i = tid; i < 4 * 256; i += kSortThreads) (&s_wcnt[0][0])[i] = 0u;
    __syncthreads();
    const uint32_t tile = s_tile;
    const uint32_t epoch = ctl->epoch;
    const uint32_t tile_base = tile * (uint32_t)kSortTile;
    const uint32_t wbase = tile_base + (uint32_t)wave * (kWave * kSortItems);

    // Striped load: item k of lane l is element wbase + 64k + l, so (k, l) order = input order.
    uint32_t keys[kSortItems], vals[kSortItems], rank[kSortItems];
#pragma unroll
    for (int k = 0; k < kSortItems; k++) {
        uint32_t idx = wbase + (uint32_t)(k * kWave + lane);
        bool v = idx < n;
        keys[k] = v ? kin[idx] : 0u;
        vals[k] = v ? (vin ? vin[idx] : idx) : 0u;
    }

    // Rank within the wave.  Out-of-range slots take the largest digit so they sort after every
    // real key of the tile and never shift a real key's rank.
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
    for (int k = 0; k < kSortItems; k++) {
        uint32_t idx = wbase + (uint32_t)(k * kWave + lane);
        uint32_t d = idx < n ? (keys[k] >> shift) & mask : mask;
        uint64_t peers = ~0ull;
        for (uint32_t b = 0; b < pbits; b++) {
            bool bit = (d >> b) & 1u;
            uint64_t bal = __ballot(bit);
            peers &= bit ? bal : ~bal;
        }
        uint32_t before = s_wcnt[wave][d];
        uint32_t below = (uint32_t)__popcll(peers & lt);
        bool leader = (peers >> lane) == 1ull;  // highest lane of its digit group
        rank[k] = before + below;
        if (leader) s_wcnt[wave][d] = before + (uint32_t)__popcll(peers);
    }
    __syncthreads();

    // Per digit (one thread each): tile count, per-wave offsets, tile-local digit start, global
    // digit start, look-back.
    const uint32_t d = (uint32_t)tid;
    uint32_t c0 = s_wcnt[0][d], c1 = s_wcnt[1][d], c2 = s_wcnt[2][d], c3 = s_wcnt[3][d];
    uint32_t cnt = c0 + c1 + c2 + c3;
    uint64_t* my = lookback + (size_t)tile * 256u + d;
    if (tile == 0) lb_store(my, lb_word(kLbInclusive, epoch, cnt));
    else lb_store(my, lb_word(kLbAggregate, epoch, cnt));
    __syncthreads();  // everyone has read s_wcnt before it is overwritten
    s_wcnt[0][d] = 0u;
    s_wcnt[1][d] = c0;
    s_wcnt[2][d] = c0 + c1;
    s_wcnt[3][d] = c0 + c1 + c2;
    uint32_t total;
    uint32_t dstart = block256_exclusive_scan(cnt, s_scan, &total);
    uint32_t ghist = d <= mask ? ctl->hist[pass][d] : 0u;
    uint32_t gstart = block256_exclusive_scan(ghist, s_scan, &total);

    uint32_t prefix = 0;
    if (tile > 0) {
        uint32_t t = tile - 1u, spins = 0;
        for (;;) {
            uint64_t w = lb_load(lookback + (size_t)t * 256u + d);
            uint64_t st = w & (3ull << 62);
            if (st != 0 && ((uint32_t)(w >> 32) & kEpochMask) == epoch) {
                prefix += (uint32_t)w;
                if (st == kLbInclusive) break;
                if (t == 0) {  // tile 0 always publishes inclusive; never walk below it
                    atomicOr(&ctl->error, 2u);
                    break;
                }
                t--;
            } else {
                if (++spins >= kSpinLimit) {
                    atomicOr(&ctl->error, 1u);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        lb_store(my, lb_word(kLbInclusive, epoch, prefix + cnt));
    }
    s_dstart[d] = dstart;
    s_gbase[d] = gstart + prefix - dstart;
    __syncthreads();

    // Stage the tile in digit order.
#pragma unroll
    for (int k = 0; k < kSortItems; k++) {
        uint32_t idx = wbase + (uint32_t)(k * kWave + lane);
        uint32_t dk = idx < n ? (keys[k] >> shift) & mask : mask;
        uint32_t pos = s_dstart[dk] + s_wcnt[wave][dk] + rank[k];
        s_keys[pos] = keys[k];
        s_vals[pos] = vals[k];
    }
    __syncthreads();

    // Coalesced scatter: consecutive slots of one digit go to consecutive global indices.
    const uint32_t valid = n - tile_base < (uint32_t)kSortTile ? n - tile_base : (uint32_t)kSortTile;
#pragma unroll
    for (int k = 0; k < kSortItems; k++) {
        uint32_t i = (uint32_t)(k * kSortThreads + tid);
        if (i < valid) {
            uint32_t key = s_keys[i];
            uint32_t dst = s_gbase[(key >> shift) & mask] + i;
            if (dst < n) {  // always true when the histograms are consistent
                if (kout) kout[dst] = key;
                vout[dst] = s_vals[i];
            }
        }
    }
}

hipError_t launch_sort_passes(fh_ctx* c, const uint32_t* k0, const uint32_t* v0, uint32_t* kfin,
                              uint32_t* vfin, uint32_t n, uint32_t num_bits) {
    const uint32_t passes = passes_for_bits(num_bits);
    const uint32_t tiles = ceil_div(n, (uint32_t)kSortTile);
    const uint32_t* kin = k0;
    const uint32_t* vin = v0;
    for (uint32_t p = 0; p < passes; p++) {
        bool last = p + 1 == passes;
        uint32_t* kout = last ? kfin : ((p & 1u) ? c->kb : c->ka);
        uint32_t* vout = last ? vfin : ((p & 1u) ? c->vb : c->va);
        uint32_t pbits = min(8u, num_bits - 8u * p);
        uint64_t* lb = c->sort_lb + (size_t)p * c->max_sort_tiles * 256u;
        tbeg(c, KID_SORT);
        k_onesweep<<<tiles, kSortThreads, 0, c->stream>>>(kin, vin, kout, vout, c->ctl, p, lb, n,
                                                          8u * p, pbits);
        tend(c, KID_SORT);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        kin = kout;
        vin = vout;
    }
    return hipSuccess;
}

}  // namespace fh
