// fh_sort.hip -- stable LSD radix sort of (key, value) pairs for gfx950.
//
// Replaces RadixSorter::sort (forge-runtime/src/radix_sort.rs:79-220), whose 4-bit passes
// re-read every earlier block's histogram per block and every earlier key per key.  Design:
//   k_begin        bump the look-back epoch, clear histograms and counters, zero the 32-bit
//                  look-back words of the coming sort
//   k_hist_keys /  one read of the keys builds the digit histograms of ALL passes into
//   k_hash_hist    per-workgroup partial rows (k_hash_hist computes the keys from positions on
//                  the fly: the hash of HashGrid::build, hashgrid.rs:89-92, fused)
//   k_hist_reduce  sums the partial rows into the histograms and marks the passes whose digit
//                  is equal for every key; for small sorts also the first pass's tile prefixes
//                  (its input order is the rows' order), so that pass needs no look-back
//   sort_plan      decides which passes run (an identity pass is skipped), in every workgroup
//                  of every pass from the marks
//   k_onesweep     one kernel per pass: an 8192-key tile per 512-lane workgroup, ranked with
//                  64-lane ballot match-any, digit offsets from a decoupled look-back over
//                  dynamically numbered tiles, then staged in LDS in digit order (keys, then
//                  values through the same buffer) so the global scatter writes contiguous runs
//   k_sort_finish  copies the result of a one-pass sort in place back from scratch
// Digits are 8 bits (256 bins), or 10 bits (1024 bins) for keys of 17..20 bits below
// kWideMaxN keys (digits_for): a pass over a million keys is bound by its look-back chain
// across the tiles, not by its bytes, so two 10-bit passes beat three 8-bit ones -- provided a
// tile's 1024 look-back words move as 512 contiguous 64-bit pairs (two digits per thread, one
// status per pair), not as 1024 strided 32-bit words.
// Stability: within a tile the rank of a key counts the equal digits before it in input order
// (earlier items, earlier lanes, earlier waves); across tiles the look-back prefix counts the
// equal digits of all earlier tiles.  Equal keys therefore keep their input order, which is
// the `sort_by_key` contract of tests/radix_sort_test.rs:111-127.
//
// Device-wide atomics are performed past the per-XCD L2 on this part, so the design keeps them
// few and apart: per-workgroup histogram rows instead of global bin atomics, 32-bit look-back
// words (a poll moves half the bytes of a 64-bit epoch word), and every hot counter on a line
// of its own (Control).
#include <type_traits>

#include "fh_internal.hpp"

namespace fh {

// ---------------------------------------------------------------------------------------------
// Start of a sort (or of a hash-grid rebuild), done by the histogram kernel that every sort
// begins with: bump the epoch, clear the histograms and counters (workgroup 0), zero the 32-bit
// look-back words of the coming passes (grid-stride).  Nothing in the histogram kernel reads
// what it clears; the kernels that do come later on the stream.
struct Begin {
    Control* ctl;  // null: no start-of-sort work in this launch
    uint32_t* lb;
    uint32_t lb_words;
};

__device__ __forceinline__ void begin_work(const Begin& b) {
    if (!b.ctl) return;
    const uint32_t t = threadIdx.x;
    Control* ctl = b.ctl;
    if (blockIdx.x == 0) {
        for (uint32_t i = t; i < kDigitSlots; i += blockDim.x) ctl->hist[i] = 0u;
        if (t == 0) {
            uint32_t e = (ctl->epoch + 1u) & kEpochMask;
            ctl->epoch = e ? e : 1u;
            for (int p = 0; p < kMaxPasses; p++) ctl->tile_ctr[p].v = 0u;
            ctl->scan_ctr.v = 0u;
            for (int q = 0; q < kHeavyLists; q++) ctl->heavy_count[q].v = 0u;
            ctl->collapse_count.v = 0u;
            ctl->big_count.v = 0u;
            ctl->triv.v = 0u;
        }
    }
    for (uint32_t i = blockIdx.x * blockDim.x + t; i < b.lb_words; i += gridDim.x * blockDim.x)
        b.lb[i] = 0u;
}

// The look-back words of the passes of a sort of n keys: pass p's tiles take words
// [p * tiles * bins, (p + 1) * tiles * bins) (counted here with the small tile, which bounds the
// large one's count).
static Begin make_begin(fh_ctx* c, bool begin, uint32_t n, uint32_t num_bits) {
    if (!begin) return Begin{nullptr, nullptr, 0u};
    const Digits L = digits_for(num_bits, n);
    const uint32_t words =
        n && num_bits ? L.passes * ceil_div(n, (uint32_t)kSortTile) * (1u << L.bits) : 0u;
    return Begin{c->ctl, c->sort_lb, words};
}

// ---------------------------------------------------------------------------------------------
// Histograms.  Each workgroup counts into per-wave LDS histograms; a wave whose valid lanes all
// hold the same digit (skewed digits: c1's top byte is always 0) adds its population with one
// LDS atomic instead of 64 conflicting ones.  Digit p of key k is bits [DB p, DB p + DB) of k,
// the last pass's digit masked by `top`.  A wave's histograms are P rows of 2^DB bins.
__device__ __forceinline__ void hist_add(uint32_t* h, uint32_t d, bool valid) {
    const uint32_t d0 = __builtin_amdgcn_readfirstlane(d);
    const uint64_t other = __ballot(valid && d != d0);
    if (other == 0ull) {
        const uint64_t act = __ballot(valid);
        if ((threadIdx.x & 63u) == 0u && act) atomicAdd(&h[d0], (uint32_t)__popcll(act));
    } else if (valid) {
        atomicAdd(&h[d], 1u);
    }
}

// P = number of passes (compile time, so the pass loop unrolls); top = mask of the last pass.
template <int P, int DB>
__device__ __forceinline__ void count_key(uint32_t* sh, uint32_t k, bool valid, uint32_t top) {
    constexpr uint32_t NB = 1u << DB;
#pragma unroll
    for (int p = 0; p < P; p++)
        hist_add(sh + p * NB, (k >> (DB * p)) & (p == P - 1 ? top : NB - 1u), valid);
}

// A full chunk of this thread's kHistItems keys.  Per pass, a wave whose 64 x kHistItems keys
// all share one digit (c1's top byte; c3's top digit in most waves) adds their number with one
// atomic; otherwise every key adds 1, with no per-key uniformity test.  `tb` = bits of the last
// pass's digit.
template <int P, int DB>
__device__ __forceinline__ void count_chunk(uint32_t* sh, const uint32_t (&k)[kHistItems],
                                            uint32_t tb) {
    constexpr uint32_t NB = 1u << DB;
#pragma unroll
    for (int p = 0; p < P; p++) {
        const uint32_t w = p == P - 1 ? tb : (uint32_t)DB;
        uint32_t* h = sh + p * NB;
        const uint32_t d0 =
            __builtin_amdgcn_readfirstlane(__builtin_amdgcn_ubfe(k[0], DB * p, w));
        uint32_t diff = 0;
#pragma unroll
        for (int j = 0; j < kHistItems; j++) diff |= __builtin_amdgcn_ubfe(k[j], DB * p, w) ^ d0;
        if (__ballot(diff != 0u) == 0ull) {
            if ((threadIdx.x & 63u) == 0u) atomicAdd(&h[d0], 64u * kHistItems);
        } else {
#pragma unroll
            for (int j = 0; j < kHistItems; j++)
                atomicAdd(&h[__builtin_amdgcn_ubfe(k[j], DB * p, w)], 1u);
        }
    }
}

// Per-workgroup LDS histograms: one copy per pair of waves (four copies, one per wave, cost the
// c3 substep 0.4 us more in clearing and summing).
constexpr int kHistCopies = kHistThreads / 128;
// Write this workgroup's row of partial histograms (all bins of every pass, P * 2^DB slots).
template <int S>
__device__ __forceinline__ void write_row(uint32_t (*sh)[S], uint32_t* part) {
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < (uint32_t)S; i += kHistThreads) {
        uint32_t t = 0;
#pragma unroll
        for (int q = 0; q < kHistCopies; q++) t += sh[q][i];
        part[(size_t)blockIdx.x * kDigitSlots + i] = t;
    }
}

template <int P, int DB>
__global__ __launch_bounds__(kHistThreads) void k_hist_keys(const uint32_t* __restrict__ keys,
                                                            uint32_t n, uint32_t top,
                                                            uint32_t* __restrict__ part,
                                                            Begin bg) {
    constexpr int S = P << DB;  // slots of one wave's histograms
    __shared__ uint32_t sh[kHistCopies][S];
    const uint32_t wave = threadIdx.x >> 6;
    begin_work(bg);
    for (uint32_t i = threadIdx.x; i < (uint32_t)kHistCopies * S; i += kHistThreads) (&sh[0][0])[i] = 0u;
    __syncthreads();
    const uint32_t chunks = ceil_div(n, (uint32_t)kHistChunk);
    // Striped chunk loads (item j of thread t is key base + 256 j + t); the loads of the next
    // chunk are issued before the current one is counted.
    uint32_t cur[kHistItems], nxt[kHistItems];
    uint32_t c = blockIdx.x;
#pragma unroll
    for (int j = 0; j < kHistItems; j++) {
        const uint32_t i = c * kHistChunk + j * kHistThreads + threadIdx.x;
        cur[j] = keys[min(i, n - 1u)];  // n >= 2; loads past n are never counted
    }
    for (; c < chunks; c += gridDim.x) {
        const uint32_t cn = c + gridDim.x;
#pragma unroll
        for (int j = 0; j < kHistItems; j++) {
            const uint32_t i = cn * kHistChunk + j * kHistThreads + threadIdx.x;
            nxt[j] = keys[min(i, n - 1u)];
        }
        if ((c + 1u) * kHistChunk <= n) {  // workgroup-uniform
            count_chunk<P, DB>(sh[wave >> 1], cur, (uint32_t)__popc(top));
        } else {
#pragma unroll
            for (int j = 0; j < kHistItems; j++) {
                const uint32_t i = c * kHistChunk + j * kHistThreads + threadIdx.x;
                count_key<P, DB>(sh[wave >> 1], cur[j], i < n, top);
            }
        }
#pragma unroll
        for (int j = 0; j < kHistItems; j++) cur[j] = nxt[j];
    }
    write_row<S>(sh, part);
}

template <int P, int DB>
__global__ __launch_bounds__(kHistThreads) void k_hash_hist(
    const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ z,
    uint32_t stride, uint32_t n, GridDesc g, uint32_t top, uint32_t* __restrict__ keys_out,
    uint32_t* __restrict__ vals_out, uint32_t* __restrict__ part, Begin bg) {
    constexpr int S = (P > 0 ? P : 1) << DB;
    __shared__ uint32_t sh[kHistCopies][S];
    const uint32_t wave = threadIdx.x >> 6;
    begin_work(bg);
    if (P > 0) {
        for (uint32_t i = threadIdx.x; i < (uint32_t)kHistCopies * S; i += kHistThreads) (&sh[0][0])[i] = 0u;
        __syncthreads();
    }
    const uint32_t chunks = ceil_div(n, (uint32_t)kHistChunk);
    for (uint32_t c = blockIdx.x; c < chunks; c += gridDim.x) {
        uint32_t k[kHistItems];
#pragma unroll
        for (int j = 0; j < kHistItems; j++) {
            const uint32_t i = c * kHistChunk + j * kHistThreads + threadIdx.x;
            k[j] = 0u;
            if (i < n) {
                const size_t o = (size_t)i * stride;
                k[j] = sort_key_of(x[o], y[o], z[o], g);
            }
        }
#pragma unroll
        for (int j = 0; j < kHistItems; j++) {
            const uint32_t i = c * kHistChunk + j * kHistThreads + threadIdx.x;
            if (i < n) {
                if (keys_out) keys_out[i] = k[j];
                if (vals_out) vals_out[i] = i;
            }
        }
        if (P > 0) {
            if ((c + 1u) * kHistChunk <= n) {  // workgroup-uniform
                count_chunk<P, DB>(sh[wave >> 1], k, (uint32_t)__popc(top));
            } else {
#pragma unroll
                for (int j = 0; j < kHistItems; j++) {
                    const uint32_t i = c * kHistChunk + j * kHistThreads + threadIdx.x;
                    count_key<P, DB>(sh[wave >> 1], k[j], i < n, top);
                }
            }
        }
    }
    if (P > 0) write_row<S>(sh, part);
}

// Sum the partial rows: workgroup (r, b) adds rows r*R .. r*R+R-1 of histogram slots
// 256 b .. 256 b + 255 into the histograms.  (No fence / last-workgroup election here: an
// agent-scope release on this part writes the L2 back, which costs tens of microseconds per
// workgroup; the decision about the passes is a separate one-workgroup kernel, the kernel
// boundary gives the visibility.)
// First-pass prefixes (pre != null: a small sort, whose histogram rows are its 4096-key chunks,
// rpt of them per first-pass tile): for the first pass's digits (slots < nb0), this workgroup's
// rows are the tiles of group g, and it also writes each tile's exclusive prefix within them,
// pre[t * nb0 + d], and their sum, pre[(tiles + g) * nb0 + d].  The first pass of the sort then
// takes its tiles' global prefixes from these instead of a look-back across the tiles.
static_assert(kPreItems * kSortThreads == kHistChunk && kSortTile == 2 * kHistChunk &&
                  kHistRowsPerReduce >= 2 && (kHistRowsPerReduce & (kHistRowsPerReduce - 1)) == 0,
              "first-pass prefixes: one or two histogram chunks per tile, whole tiles per group");
// RPT (rows per first-pass tile, 1 or 2) is a template argument: with a run-time one the
// unrolled row loop no longer overlaps its loads (c2's build 0.100 -> 0.112 ms).
template <uint32_t RPT>
__global__ __launch_bounds__(256) void k_hist_reduce(const uint32_t* __restrict__ part,
                                                     uint32_t rows, uint32_t slot_blocks,
                                                     Control* ctl, uint32_t* __restrict__ pre,
                                                     uint32_t nb0, uint32_t tiles, uint32_t n,
                                                     uint32_t rpr) {
    const uint32_t b = blockIdx.x % slot_blocks, g = blockIdx.x / slot_blocks;
    const uint32_t r0 = g * rpr;
    const uint32_t slot = b * 256u + threadIdx.x;
    const uint32_t r1 = min(rows, r0 + rpr);
    uint32_t s = 0;
    if (pre && slot < nb0) {  // uniform per workgroup (nb0 is a multiple of 256)
#pragma unroll 8
        for (uint32_t r = r0; r < r1; r++) {
            if (!((r - r0) & (RPT - 1u))) pre[(size_t)(r / RPT) * nb0 + slot] = s;
            s += part[(size_t)r * kDigitSlots + slot];
        }
        pre[((size_t)tiles + g) * nb0 + slot] = s;
    } else {
#pragma unroll 8
        for (uint32_t r = r0; r < r1; r++) s += part[(size_t)r * kDigitSlots + slot];
    }
    if (s) {
        // the add that completes a bin holding every key marks its pass as the identity (exactly
        // one add sees the count reach n: counts only grow)
        if (atomicAdd(&ctl->hist[slot], s) + s == n) atomicOr(&ctl->triv.v, 1u << (slot / nb0));
    }
}

// The passes that run (one bit per pass), derived by every workgroup of every pass from the
// trivial-pass bits k_hist_reduce left (the same function of the same word, so all agree).  A
// pass whose digit is equal for every key (one histogram bin holds all n keys) is the identity
// and is skipped.  Two adjustments leave the result in (kfin, vfin) without a copy kernel: when
// no pass moves keys and the sort is out of place, pass 0 runs (a stable copy: its digit is
// constant); when exactly one pass moves keys in place (it has to write scratch) and the sort
// has another pass, that pass runs as well (also a copy), so the second of the two writes back
// in place.  Only one-pass sorts in place keep k_sort_finish (which reads ctl->plan, written by
// pass 0).
__device__ __forceinline__ uint32_t sort_plan(const Control* __restrict__ ctl, uint32_t passes,
                                              bool in_place) {
    uint32_t plan = ~ctl->triv.v & ((1u << passes) - 1u);
    if (plan == 0u && !in_place) {
        plan = 1u;
    } else if (__popc(plan) == 1 && in_place && passes >= 2u) {
        const uint32_t p = (uint32_t)(__ffs(plan) - 1);
        plan |= 1u << (p > 0u ? p - 1u : 1u);
    }
    return plan;
}


// The first-pass prefix buffer of a sort of n keys, or null (sorts of more than 4,194,304 keys,
// whose histogram workgroups take several chunks each).
static uint32_t* first_pass_pre(fh_ctx* c, uint32_t n) {
    // the prefixes need one partial histogram row per 4096-key chunk of the input
    return n <= (uint32_t)kHistBlocks * kHistChunk ? c->sort_pre : nullptr;
}

hipError_t launch_hist_reduce(fh_ctx* c, uint32_t rows, uint32_t slots, uint32_t n,
                              uint32_t nb0) {
    // groups of kHistRowsPerReduce rows where the first pass takes its prefixes from them, else
    // of kHistRowsPlain rows (more workgroups for the plain sums)
    uint32_t* const pre = first_pass_pre(c, n);
    const uint32_t rpr = pre ? (uint32_t)kHistRowsPerReduce : (uint32_t)kHistRowsPlain;
    const uint32_t groups = ceil_div(rows, rpr);
    const uint32_t slot_blocks = slots / 256u;  // slots = passes * bins, bins >= 256
    const auto kernel = pre_rows_per_tile(n) == 1u ? k_hist_reduce<1> : k_hist_reduce<2>;
    kernel<<<groups * slot_blocks, 256, 0, c->stream>>>(
        c->hist_part, rows, slot_blocks, c->ctl, pre, nb0,
        ceil_div(n, (uint32_t)kHistChunk * pre_rows_per_tile(n)), n, rpr);
    return hipGetLastError();
}

static uint32_t hist_blocks(uint32_t n) {
    uint32_t b = ceil_div(n, (uint32_t)kHistChunk);
    if (b < 1) b = 1;
    if (b > (uint32_t)kHistBlocks) b = kHistBlocks;
    return b;
}

hipError_t launch_hist_keys(fh_ctx* c, const uint32_t* keys, uint32_t n, uint32_t num_bits,
                            bool begin) {
    if (begin) {
        const hipError_t e = note_begin(c);
        if (e != hipSuccess) return e;
    }
    const Digits L = digits_for(num_bits, n);
    const uint32_t blocks = hist_blocks(n), top = (1u << L.top_bits) - 1u;
    const Begin bg = make_begin(c, begin, n, num_bits);
    uint32_t* part = c->hist_part;
    tbeg(c, KID_HIST);
    if (L.bits == kWideDigitBits) {  // 17..20 bits: two passes
        k_hist_keys<2, kWideDigitBits><<<blocks, kHistThreads, 0, c->stream>>>(keys, n, top, part, bg);
    } else {
        switch (L.passes) {
            case 1: k_hist_keys<1, 8><<<blocks, kHistThreads, 0, c->stream>>>(keys, n, top, part, bg); break;
            case 2: k_hist_keys<2, 8><<<blocks, kHistThreads, 0, c->stream>>>(keys, n, top, part, bg); break;
            case 3: k_hist_keys<3, 8><<<blocks, kHistThreads, 0, c->stream>>>(keys, n, top, part, bg); break;
            default: k_hist_keys<4, 8><<<blocks, kHistThreads, 0, c->stream>>>(keys, n, top, part, bg); break;
        }
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = launch_hist_reduce(c, blocks, L.passes << L.bits, n, 1u << L.bits);
    tend(c, KID_HIST);
    return e;
}

hipError_t launch_hash_hist(fh_ctx* c, const float* x, const float* y, const float* z,
                            uint32_t stride, uint32_t n, const GridDesc& g, uint32_t num_bits,
                            uint32_t* keys_out, uint32_t* vals_out, bool begin) {
    if (begin) {
        const hipError_t e = note_begin(c);
        if (e != hipSuccess) return e;
    }
    const Digits L = digits_for(num_bits, n);
    const uint32_t blocks = hist_blocks(n), top = num_bits ? (1u << L.top_bits) - 1u : 0u;
    const Begin bg = make_begin(c, begin, n, num_bits);
    uint32_t* part = c->hist_part;
    tbeg(c, KID_HASH);
    if (num_bits > 0 && L.bits == kWideDigitBits) {
        k_hash_hist<2, kWideDigitBits><<<blocks, kHistThreads, 0, c->stream>>>(x, y, z, stride, n, g, top, keys_out, vals_out, part, bg);
    } else {
        switch (L.passes) {
            case 0: k_hash_hist<0, 8><<<blocks, kHistThreads, 0, c->stream>>>(x, y, z, stride, n, g, top, keys_out, vals_out, part, bg); break;
            case 1: k_hash_hist<1, 8><<<blocks, kHistThreads, 0, c->stream>>>(x, y, z, stride, n, g, top, keys_out, vals_out, part, bg); break;
            case 2: k_hash_hist<2, 8><<<blocks, kHistThreads, 0, c->stream>>>(x, y, z, stride, n, g, top, keys_out, vals_out, part, bg); break;
            case 3: k_hash_hist<3, 8><<<blocks, kHistThreads, 0, c->stream>>>(x, y, z, stride, n, g, top, keys_out, vals_out, part, bg); break;
            default: k_hash_hist<4, 8><<<blocks, kHistThreads, 0, c->stream>>>(x, y, z, stride, n, g, top, keys_out, vals_out, part, bg); break;
        }
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && num_bits > 0)
        e = launch_hist_reduce(c, blocks, L.passes << L.bits, n, 1u << L.bits);
    tend(c, KID_HASH);
    return e;
}

// ---------------------------------------------------------------------------------------------
// Buffers of one sort.  A sort is either in place ((kfin, vfin) == (k0, v0)) or entirely out of
// place (launch_sort_passes checks).  Pass j of the passes that run (the plan) reads the output
// of pass j-1 (pass 0: k0 / v0) and writes, alternately, scratch a and b; the last one writes
// (kfin, vfin) unless it is also the first and the sort is in place, in which case it writes a
// (sort_plan avoids that case for sorts of more than one pass).
struct SortIO {
    const uint32_t* k0;
    const uint32_t* v0;  // null: values are the indices 0..n-1
    uint32_t* ka;
    uint32_t* va;
    uint32_t* kb;
    uint32_t* vb;
    uint32_t* kfin;      // null: keys are not needed in the output
    uint32_t* vfin;
    uint32_t* rank;      // non-null: the last pass also writes rank[value] = output index
    uint32_t passes;     // passes of the sort
    uint32_t in_place;
    const uint32_t* pre; // first-pass tile prefixes (k_hist_reduce), or null
    uint32_t tiles;      // tiles of the first pass (the group sums follow them in pre)
    uint32_t group_shift; // log2 of the first-pass tiles per group of pre
    uint32_t kshift;     // the last pass writes key >> kshift to kfin (sub-cell bits dropped)
};

struct PassBufs {
    const uint32_t* kin;
    const uint32_t* vin;
    uint32_t* kout;
    uint32_t* vout;
};

__device__ __forceinline__ bool sort_in_place(const SortIO& io) {
    return io.kfin != nullptr && io.kfin == io.k0;
}

__device__ __forceinline__ PassBufs pass_bufs(SortIO io, uint32_t plan, uint32_t pass) {
    const uint32_t j = (uint32_t)__popc(plan & ((1u << pass) - 1u));
    const bool last = (plan >> (pass + 1u)) == 0u;
    PassBufs b;
    b.kin = j == 0 ? io.k0 : ((j & 1u) ? io.ka : io.kb);
    b.vin = j == 0 ? io.v0 : ((j & 1u) ? io.va : io.vb);
    if (last && !(j == 0 && sort_in_place(io))) {
        b.kout = io.kfin;
        b.vout = io.vfin;
    } else {
        b.kout = (j & 1u) ? io.kb : io.ka;
        b.vout = (j & 1u) ? io.vb : io.va;
    }
    return b;
}

// Branch-free 64-lane match of a DB-bit digit: bit l of the result is set iff lane l holds the
// same digit.  m is 0 or all ones per lane (sign-extended digit bit); ~(ballot ^ m) keeps the
// lanes that agree with this lane on that bit.
// Per bit: one signed bit-field extract (m), one compare writing the ballot, and one 3-input
// bitwise op per half (acc & ~(ballot ^ m), truth table 0x90 over (acc, ballot, m)): 4 VALU
// per bit.  Left to itself the compiler re-associates the chain into xors and or3s and derives
// the compare from a separate shift (6 per bit).
template <int DB>
__device__ __forceinline__ void match_digit(uint32_t d, uint32_t& lo, uint32_t& hi) {
    lo = 0xFFFFFFFFu;
    hi = 0xFFFFFFFFu;
#pragma unroll
    for (int b = 0; b < DB; b++) {
        // m is produced by an opaque v_bfe_i32 so the ballot compares it with zero directly
        // (otherwise the compiler derives the condition with a separate shift).
        uint32_t m;
        asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(m) : "v"(d), "n"(b));
        const uint64_t bal = __ballot(m != 0u);
        lo = __builtin_amdgcn_bitop3_b32(lo, (uint32_t)bal, m, 0x90);
        hi = __builtin_amdgcn_bitop3_b32(hi, (uint32_t)(bal >> 32), m, 0x90);
    }
}

#ifndef FH_LB_WIN
#define FH_LB_WIN 4
#endif
constexpr int kLbWin = FH_LB_WIN;  // look-back words loaded per round trip

// Load of item k of this lane (element wbase + 64k + lane): unchecked in full tiles.
template <bool Full>
__device__ __forceinline__ uint32_t item_load(const uint32_t* __restrict__ p, uint32_t idx,
                                              uint32_t n, uint32_t pad) {
    return (Full || idx < n) ? p[idx] : pad;
}

template <bool Full, int Items>
__device__ __forceinline__ void load_items(const uint32_t* __restrict__ p, uint32_t wbase,
                                           int lane, uint32_t n, uint32_t pad,
                                           uint32_t (&v)[Items]) {
#pragma unroll
    for (int k = 0; k < Items; k++)
        v[k] = item_load<Full>(p, wbase + (uint32_t)(k * kWave + lane), n, pad);
}

// Values of the items: loaded, or the element indices when the input values are implicit.
template <bool Full, int Items>
__device__ __forceinline__ void load_vals(const uint32_t* __restrict__ vin, uint32_t wbase,
                                          int lane, uint32_t n, uint32_t (&v)[Items]) {
    if (vin) {
        load_items<Full, Items>(vin, wbase, lane, n, 0u, v);
    } else {
#pragma unroll
        for (int k = 0; k < Items; k++) v[k] = wbase + (uint32_t)(k * kWave + lane);
    }
}

// Look-back words of one tile for the DPT digits a thread owns, all with status `st`: one
// 32-bit word, or -- two digits per thread -- both words in one 64-bit store, so that the pair
// always carries one status and a single walk serves both digits (and the wave's loads stay
// contiguous: lane l reads bytes 8l .. 8l + 7 of the tile's row).
template <int DPT>
__device__ __forceinline__ void lb_publish(uint32_t* w, uint32_t st, const uint32_t (&v)[DPT]) {
    static_assert(DPT == 1 || DPT == 2, "one or two digits per thread");
    if constexpr (DPT == 1) {
        __hip_atomic_store(w, st | v[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        __hip_atomic_store((uint64_t*)w, (uint64_t)(st | v[0]) | ((uint64_t)(st | v[1]) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Windowed decoupled look-back of tile `tile` (> 0) for the thread's digits, whose words are
// w[t * NB] for tile t: the words of the kLbWin tiles below `t` are loaded together (one round
// trip instead of kLbWin), then consumed nearest first: aggregates are summed into prefix until
// an inclusive prefix ends the walk; a word not yet published stops the window and is polled
// again.  Tiles below 0 are never read (tile 0 publishes inclusive); a bounded number of polls
// keeps every wave finite and raises the device error flag instead.
template <int DPT>
__device__ __forceinline__ void lb_walk(const uint32_t* __restrict__ w, uint32_t NB, uint32_t tile,
                                        uint32_t (&prefix)[DPT], Control* ctl) {
    using Word = typename std::conditional<DPT == 1, uint32_t, uint64_t>::type;
    uint32_t t = tile, spins = 0;  // the walk continues at tile t - 1
    const uint32_t limit = ctl->spin_limit ? ctl->spin_limit : kSpinLimit;
    for (;;) {
        Word x[kLbWin];
#pragma unroll
        for (int j = 0; j < kLbWin; j++)
            x[j] = t > (uint32_t)j ? __hip_atomic_load((const Word*)(w + (size_t)(t - 1u - j) * NB),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : (Word)0;
        uint32_t adv = 0;
        bool done = false, stop = false;
#pragma unroll
        for (int j = 0; j < kLbWin; j++) {
            const uint32_t st = (uint32_t)x[j] & (3u << 30);
            if (!stop && !done && t > (uint32_t)j && st != 0u) {
                prefix[0] += (uint32_t)x[j] & 0x3FFFFFFFu;
                if constexpr (DPT == 2) prefix[1] += (uint32_t)(x[j] >> 32) & 0x3FFFFFFFu;
                adv++;
                done = st == kLb32Inclusive;
            } else {
                stop = true;
            }
        }
        if (done) break;
        t -= adv;
        if (t == 0) {  // tile 0 always publishes inclusive; never walk below it
            atomicOr(&ctl->error.v, 2u);
            break;
        }
        // every poll counts (a walk over the most tiles of a context needs < 2^15 of them)
        if (++spins >= limit) {
            atomicOr(&ctl->error.v, 1u);
            break;
        }
        if (adv == 0) __builtin_amdgcn_s_sleep(1);
    }
}

// Items = keys per thread: a tile holds Items * kSortThreads keys (kSortItems for small sorts
// and 10-bit digits, kSortItemsLarge for 8-bit digits from kSortLargeN keys on: longer per-digit runs in the scatter and half as
// many look-back words per key, at two workgroups per CU).  DB = digit bits: 2^DB bins; in the
// per-digit phases thread t owns digits t * DPT .. t * DPT + DPT - 1 (the first 256 threads,
// one digit each, for 8-bit digits; every thread, two digits each, for 10-bit ones).
template <int Items, int DB>
__global__ __launch_bounds__(kSortThreads, Items > kSortItems ? 2 : FH_SORT_MINB) void k_onesweep(
    SortIO io, Control* ctl, uint32_t pass, uint32_t* __restrict__ lookback, uint32_t n,
    uint32_t shift, uint32_t pbits) {
    constexpr uint32_t kTile = (uint32_t)(Items * kSortThreads);
    constexpr uint32_t NB = 1u << DB;
    constexpr int DPT = NB > (uint32_t)kSortThreads ? (int)(NB / kSortThreads) : 1;
    constexpr uint32_t kOwners = NB / DPT;  // threads that own digits
    __shared__ uint32_t s_buf[kTile];
    __shared__ uint32_t s_wcnt[kSortWaves][NB];  // per-wave digit counts, then wave offsets
    __shared__ uint32_t s_gbase[NB];             // global index of tile slot 0 of digit d
    __shared__ uint32_t s_scan[kSortWaves];
    __shared__ uint32_t s_tile;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t plan = sort_plan(ctl, io.passes, io.in_place != 0u);
    if (pass == 0u && blockIdx.x == 0u && tid == 0) ctl->plan = plan;  // for k_sort_finish
    if (!((plan >> pass) & 1u)) return;  // the pass does not run (workgroup-uniform)
    const PassBufs bf = pass_bufs(io, plan, pass);
    const bool last = (plan >> (pass + 1u)) == 0u;

    const uint32_t mask = (1u << pbits) - 1u;
    if (tid == 0) s_tile = atomicAdd(&ctl->tile_ctr[pass].v, 1u);
    for (int i = tid; i < kSortWaves * (int)NB; i += kSortThreads) (&s_wcnt[0][0])[i] = 0u;
    __syncthreads();
    const uint32_t tile = s_tile;
    const uint32_t tile_base = tile * kTile;
    const uint32_t wbase = tile_base + (uint32_t)wave * (kWave * Items);
    const bool full = n - tile_base >= kTile;  // workgroup-uniform

    // Striped key loads: item k of lane l is element wbase + 64k + l, so (k, l) order = input
    // order.  Slots past n hold digit `mask` and rank after every real key of the tile.
    uint32_t keys[Items], vals[Items], pos[Items];
    if (full) load_items<true, Items>(bf.kin, wbase, lane, n, 0xFFFFFFFFu, keys);
    else load_items<false, Items>(bf.kin, wbase, lane, n, 0xFFFFFFFFu, keys);
    const uint32_t lt_lo = lane >= 32 ? 0xFFFFFFFFu : ((1u << lane) - 1u);
    const uint32_t lt_hi = lane <= 32 ? 0u : (0xFFFFFFFFu >> (64 - lane));
    const uint32_t gt_lo = lane >= 31 ? 0u : (0xFFFFFFFFu << (lane + 1));
    const uint32_t gt_hi = lane < 31 ? 0xFFFFFFFFu : (lane == 63 ? 0u : (0xFFFFFFFFu << (lane - 31)));
#pragma unroll
    for (int k = 0; k < Items; k++) {
        const uint32_t d = (keys[k] >> shift) & mask;
        uint32_t lo, hi;
        match_digit<DB>(d, lo, hi);
        const uint32_t before = s_wcnt[wave][d];
        pos[k] = before + (uint32_t)(__popc(lo & lt_lo) + __popc(hi & lt_hi));
        if (((lo & gt_lo) | (hi & gt_hi)) == 0u)  // highest lane of its digit group
            s_wcnt[wave][d] = before + (uint32_t)(__popc(lo) + __popc(hi));
        // Materialise the rank here: left alone, the compiler defers the popcounts to the
        // staging loop and keeps every item's 64-bit match mask alive across the look-back.
        asm volatile("" : "+v"(pos[k]));
    }
    __syncthreads();

    // Per owned digit: tile count, published at once as this tile's aggregate; wave offsets;
    // tile-local digit start; global digit start.
    const bool owner = (uint32_t)tid < kOwners;
    const uint32_t d0 = (uint32_t)tid * DPT;
    uint32_t cnt[DPT], wc[DPT][kSortWaves], tsum = 0;
#pragma unroll
    for (int k = 0; k < DPT; k++) {
        cnt[k] = 0u;
        if (owner) {
#pragma unroll
            for (int w = 0; w < kSortWaves; w++) {
                wc[k][w] = s_wcnt[w][d0 + k];
                cnt[k] += wc[k][w];
            }
        }
        tsum += cnt[k];
    }
    const bool precomputed = pass == 0u && io.pre != nullptr;  // uniform
    if (owner && !precomputed)
        lb_publish<DPT>(lookback + (size_t)tile * NB + d0,
                        tile == 0 ? kLb32Inclusive : kLb32Aggregate, cnt);
    uint32_t total;
    uint32_t dstart[DPT];
    {
        uint32_t run = block_exclusive_scan<kSortWaves>(owner ? tsum : 0u, s_scan, &total);
#pragma unroll
        for (int k = 0; k < DPT; k++) {
            dstart[k] = run;
            if (owner) {
                uint32_t r = run;
#pragma unroll
                for (int w = 0; w < kSortWaves; w++) {
                    s_wcnt[w][d0 + k] = r;
                    r += wc[k][w];
                }
            }
            run += cnt[k];
        }
    }
    uint32_t gstart[DPT];
    {
        uint32_t gh[DPT], gsum = 0;
#pragma unroll
        for (int k = 0; k < DPT; k++) {
            gh[k] = (owner && d0 + k <= mask) ? ctl->hist[pass * NB + d0 + k] : 0u;
            gsum += gh[k];
        }
        uint32_t run = block_exclusive_scan<kSortWaves>(gsum, s_scan, &total);
#pragma unroll
        for (int k = 0; k < DPT; k++) {
            gstart[k] = run;
            run += gh[k];
        }
    }

    // Stage the keys in tile-local digit order (that needs only this tile's counts; the scan's
    // barriers published the wave offsets) and issue the value loads, so both overlap the
    // look-back's wait for earlier tiles.
#pragma unroll
    for (int k = 0; k < Items; k++) {
        pos[k] += s_wcnt[wave][(keys[k] >> shift) & mask];
        s_buf[pos[k]] = keys[k];
    }
    if (full) load_vals<true, Items>(bf.vin, wbase, lane, n, vals);
    else load_vals<false, Items>(bf.vin, wbase, lane, n, vals);
    __syncthreads();
    uint32_t skey[Items];
#pragma unroll
    for (int k = 0; k < Items; k++) skey[k] = s_buf[k * kSortThreads + tid];

    uint32_t prefix[DPT];
#pragma unroll
    for (int k = 0; k < DPT; k++) prefix[k] = 0u;
    if (owner && tile > 0 && precomputed) {
        // the first pass reads the input order: the tile's prefix within its group of tiles
        // plus the sums of the groups before it (k_hist_reduce)
#pragma unroll
        for (int k = 0; k < DPT; k++) prefix[k] = io.pre[(size_t)tile * NB + d0 + k];
        const uint32_t groups = tile >> io.group_shift;
#pragma unroll 8
        for (uint32_t q = 0; q < groups; q++)
#pragma unroll
            for (int k = 0; k < DPT; k++)
                prefix[k] += io.pre[((size_t)io.tiles + q) * NB + d0 + k];
    } else if (owner && tile > 0) {
        lb_walk<DPT>(lookback + d0, NB, tile, prefix, ctl);
        uint32_t inc[DPT];
#pragma unroll
        for (int k = 0; k < DPT; k++) inc[k] = prefix[k] + cnt[k];
        lb_publish<DPT>(lookback + (size_t)tile * NB + d0, kLb32Inclusive, inc);
    }
    if (owner) {
#pragma unroll
        for (int k = 0; k < DPT; k++) s_gbase[d0 + k] = gstart[k] + prefix[k] - dstart[k];
    }
    __syncthreads();

    // Scatter the keys (contiguous runs per digit), then the values through the same buffer.
    // dst < n holds whenever the histograms and look-back are consistent; the check keeps a
    // corrupted state (a spin limit hit) from writing out of bounds.
    const uint32_t valid = full ? kTile : n - tile_base;
    uint32_t dst[Items];
#pragma unroll
    for (int k = 0; k < Items; k++) {
        const uint32_t i = (uint32_t)(k * kSortThreads + tid);
        dst[k] = s_gbase[(skey[k] >> shift) & mask] + i;
        if ((full || i < valid) && dst[k] < n && bf.kout)
            bf.kout[dst[k]] = last ? skey[k] >> io.kshift : skey[k];
    }
#pragma unroll
    for (int k = 0; k < Items; k++) s_buf[pos[k]] = vals[k];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < Items; k++) {
        const uint32_t i = (uint32_t)(k * kSortThreads + tid);
        if ((full || i < valid) && dst[k] < n) {
            const uint32_t v = s_buf[i];
            bf.vout[dst[k]] = v;
            if (last && io.rank && v < n) io.rank[v] = dst[k];  // inverse permutation
        }
    }
}

// A one-pass sort in place whose pass ran wrote scratch a: copy it back.
__global__ __launch_bounds__(256) void k_sort_finish(SortIO io, const Control* ctl, uint32_t n) {
    if (!(ctl->plan & 1u)) return;
    for (uint32_t i = blockIdx.x * 256u + threadIdx.x; i < n; i += gridDim.x * 256u) {
        io.kfin[i] = io.ka[i];
        io.vfin[i] = io.va[i];
    }
}

hipError_t launch_sort_passes(fh_ctx* c, const uint32_t* k0, const uint32_t* v0, uint32_t* kfin,
                              uint32_t* vfin, uint32_t n, uint32_t num_bits, uint32_t* rank,
                              uint32_t kshift) {
    const Digits L = digits_for(num_bits, n);
    const uint32_t passes = L.passes, nb = 1u << L.bits;
    // large 8-bit sorts: 12,288-key tiles and the plan without first-pass prefixes
    const bool large = n >= kSortLargeN && L.bits != kWideDigitBits;
    const uint32_t tiles = ceil_div(n, (uint32_t)(large ? kSortTileLarge : kSortTile));
    const bool in_place = kfin != nullptr && kfin == k0;
    if (in_place ? (vfin != v0 || v0 == nullptr) : (vfin == v0 && v0 != nullptr) || !vfin)
        return hipErrorInvalidValue;  // mixed in place / out of place is not supported
    // a first pass that takes its prefixes from k_hist_reduce runs on tiles of pre_rows_per_tile
    // histogram rows: one row (kPreItems keys per thread, twice the workgroups of the later
    // passes) for up to kPreSmallMaxN keys
    const uint32_t* const pre = large ? nullptr : first_pass_pre(c, n);
    const bool one_row = pre_rows_per_tile(n) == 1u;
    const uint32_t pre_tiles = ceil_div(n, (uint32_t)kHistChunk * pre_rows_per_tile(n));
    SortIO io{k0, v0, c->ka, c->va, c->kb, c->vb, kfin, vfin, rank, passes, in_place ? 1u : 0u,
              pre, pre_tiles, (uint32_t)__builtin_ctz(kHistRowsPerReduce / pre_rows_per_tile(n)),
              kshift};
    // the second pass of such a two-pass sort takes one-row tiles as well, its look-back words
    // from word 0 (the first pass uses none, and 2 x ceil(n / kSortTile) x nb words, what
    // make_begin zeroes for two passes, hold ceil(n / kHistChunk) x nb)
    const bool one_row_both = pre && one_row && passes == 2u;
    for (uint32_t p = 0; p < passes; p++) {
        const uint32_t shift = L.bits * p, pbits = min(L.bits, num_bits - shift);
        const bool small_tiles = p == 0u ? pre && one_row : one_row_both;
        uint32_t* lb = small_tiles ? c->sort_lb : c->sort_lb + (size_t)p * tiles * nb;
        tbeg(c, KID_SORT);
        if (small_tiles && L.bits == kWideDigitBits)
            k_onesweep<kPreItems, kWideDigitBits><<<pre_tiles, kSortThreads, 0, c->stream>>>(
                io, c->ctl, p, lb, n, shift, pbits);
        else if (small_tiles)
            k_onesweep<kPreItems, 8><<<pre_tiles, kSortThreads, 0, c->stream>>>(io, c->ctl, p, lb,
                                                                               n, shift, pbits);
        else if (L.bits == kWideDigitBits)
            k_onesweep<kSortItems, kWideDigitBits><<<tiles, kSortThreads, 0, c->stream>>>(
                io, c->ctl, p, lb, n, shift, pbits);
        else if (large)
            k_onesweep<kSortItemsLarge, 8><<<tiles, kSortThreads, 0, c->stream>>>(io, c->ctl, p, lb,
                                                                                  n, shift, pbits);
        else
            k_onesweep<kSortItems, 8><<<tiles, kSortThreads, 0, c->stream>>>(io, c->ctl, p, lb, n,
                                                                             shift, pbits);
        tend(c, KID_SORT);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    if (passes == 1u && in_place) {
        uint32_t blocks = ceil_div(n, 256u * 8u);
        if (blocks > 1024) blocks = 1024;
        if (blocks < 1) blocks = 1;
        k_sort_finish<<<blocks, 256, 0, c->stream>>>(io, c->ctl, n);
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace fh
