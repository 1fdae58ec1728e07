// fh_stream.hpp -- wave-level candidate streams shared by the SPH light passes and the
// neighbour query (gfx950, wave64).
//
// A wave owns 64 consecutive sorted particles.  For one z-slab of their 3x3x3 neighbourhood,
// the particles of one home row (cy, cz) are consecutive lanes, and for each of the slab's 3
// rows the union of their neighbour ranges is one contiguous range of the sorted arrays (the
// x-adjacent cells of that row), from the first lane's begin to the last lane's end.  The
// wave's candidates are laid out as one stream -- per home-row segment in lane order, the
// unions of its rows 0, 1, 2 -- so every lane's own range of row r is one contiguous interval
// of the stream; the stream is staged through LDS a window at a time and every lane evaluates
// its own intervals clipped to the window.  A lane's candidates are visited row by row in
// stream order, i.e. in the order of its own ranges.
#pragma once

#include "fh_internal.hpp"

namespace fh {

__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, off, kWave));
    return v;
}
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = max(v, (uint32_t)__shfl_xor((int)v, off, kWave));
    return v;
}

// ---------------------------------------------------------------------------------------------
// Workgroup renumbering for the one-wave-per-item kernels (SPH light items, neighbour query).
// The dispatcher hands workgroup b to XCD b % 8, so consecutive items land on eight different
// L2s.  Mapping runs of kXcdChunk workgroups to one
// XCD keeps neighbouring sub-tiles, which read mostly the same candidate cells, on one L2 while
// every XCD still takes a share of each region of the box (balance matters more than reuse: a
// contiguous eighth of the items per XCD was slower).  The tail beyond the last whole round of
// 8 * kXcdChunk workgroups keeps its own numbers, so the mapping is a permutation of [0, nb).
constexpr uint32_t kXcdChunk = 128, kXcds = 8;
__device__ __forceinline__ uint32_t xcd_chunked(uint32_t b, uint32_t nb) {
    const uint32_t full = nb / (kXcds * kXcdChunk) * (kXcds * kXcdChunk);
    if (b >= full) return b;
    const uint32_t x = b % kXcds, i = b / kXcds;
    return ((i / kXcdChunk) * kXcds + x) * kXcdChunk + (i % kXcdChunk);
}

// Light items.  The candidates of a wave are laid out as one stream: for each home-row segment
// in lane order, the unions of its rows 0, 1, 2.  Every lane's own range of row r is then one
// contiguous interval [S[r], S[r] + cnt[r]) of the stream.  The stream is staged through the
// wave's LDS slice kWin candidates at a time, and all lanes (of every segment at once) evaluate
// their own intervals clipped to the window: segments no longer take turns.
// 256 candidates per window (c3 trajectory 407.4 -> 402.4 us per substep against 192; 128:
// slower, 320: slower on the fixed state; the kept streams then cost 132 instead of 108 bytes
// per particle)
#ifndef FH_WIN
#define FH_WIN 256
#endif
constexpr int kWin = FH_WIN;  // candidates staged per window
constexpr int kWinLoads = kWin / kWave;

struct LightStream {
    uint32_t S[3], cnt[3];  // the lane's own intervals
    uint32_t T;             // stream length (wave-uniform)
    int nseg;               // home-row segments (wave-uniform)
    // segment table: lane q < nseg holds segment q's first stream position and row unions
    // [lo[r], lo[r] + L[r])
    uint32_t cb, clo0, clo1, clo2, cL0, cL1;
};

__device__ __forceinline__ void light_stream(LightStream& L, const uint32_t b[3],
                                             const uint32_t e[3], uint32_t hr, bool in, int lane) {
    const int nin = __popcll(__ballot(in));
    const uint32_t hprev = (uint32_t)__shfl_up((int)hr, 1u, kWave);
    const bool lead = in && (lane == 0 || hprev != hr);
    const uint64_t starts = __ballot(lead);
    const uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
    const uint64_t before = starts & upto, after = starts & ~upto;
    const int leader = before ? 63 - __clzll((long long)before) : 0;
    const int last = after ? __ffsll((unsigned long long)after) - 2 : nin - 1;
    const uint32_t lo0 = (uint32_t)__shfl((int)b[0], leader, kWave);
    const uint32_t lo1 = (uint32_t)__shfl((int)b[1], leader, kWave);
    const uint32_t lo2 = (uint32_t)__shfl((int)b[2], leader, kWave);
    const uint32_t hi0 = (uint32_t)__shfl((int)e[0], last < 0 ? 0 : last, kWave);
    const uint32_t hi1 = (uint32_t)__shfl((int)e[1], last < 0 ? 0 : last, kWave);
    const uint32_t hi2 = (uint32_t)__shfl((int)e[2], last < 0 ? 0 : last, kWave);
    const uint32_t L0 = hi0 - lo0, L1 = hi1 - lo1;
    const uint32_t len = L0 + L1 + (hi2 - lo2);
    // inclusive scan of the segment lengths, counted at their leaders
    uint32_t x = lead ? len : 0u;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const uint32_t y = (uint32_t)__shfl_up((int)x, (unsigned)d, kWave);
        if (lane >= d) x += y;
    }
    L.T = (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
    const uint32_t excl = x - (lead ? len : 0u);
    const uint32_t base = (uint32_t)__shfl((int)excl, leader, kWave);
    L.S[0] = base + (b[0] - lo0);
    L.S[1] = base + L0 + (b[1] - lo1);
    L.S[2] = base + L0 + L1 + (b[2] - lo2);
#pragma unroll
    for (int r = 0; r < 3; r++) L.cnt[r] = in ? e[r] - b[r] : 0u;
    // segment table: each leader sends its segment to lane (its rank among the leaders); the
    // other lanes send to lane 63, which is a table entry only when all 64 lanes lead
    L.nseg = __popcll(starts);
    const int rk = lead ? (int)__popcll(starts & (upto >> 1)) : 63;
    const int to = rk << 2;
    L.cb = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)base);
    L.clo0 = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)lo0);
    L.clo1 = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)lo1);
    L.clo2 = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)lo2);
    L.cL0 = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)L0);
    L.cL1 = (uint32_t)__builtin_amdgcn_ds_permute(to, (int)L1);
}

// Sorted index of stream position t (< T): the last segment that starts at or before t (a
// binary search over the nseg table entries; none for one segment), then the row.
__device__ __forceinline__ uint32_t stream_index(const LightStream& L, uint32_t t) {
    uint32_t base, lo0, lo1, lo2, L0, L1;
    if (L.nseg == 1) {  // wave-uniform: the one segment's values from lane 0
        base = (uint32_t)__builtin_amdgcn_readlane((int)L.cb, 0);
        lo0 = (uint32_t)__builtin_amdgcn_readlane((int)L.clo0, 0);
        lo1 = (uint32_t)__builtin_amdgcn_readlane((int)L.clo1, 0);
        lo2 = (uint32_t)__builtin_amdgcn_readlane((int)L.clo2, 0);
        L0 = (uint32_t)__builtin_amdgcn_readlane((int)L.cL0, 0);
        L1 = (uint32_t)__builtin_amdgcn_readlane((int)L.cL1, 0);
    } else {
        int pos = 0;
        for (int step = 1 << (31 - __clz(L.nseg - 1)); step >= 1; step >>= 1) {  // uniform
            const int c = pos + step;
            const uint32_t sb = (uint32_t)__shfl((int)L.cb, c < L.nseg ? c : 0, kWave);
            if (c < L.nseg && sb <= t) pos = c;
        }
        base = (uint32_t)__shfl((int)L.cb, pos, kWave);
        lo0 = (uint32_t)__shfl((int)L.clo0, pos, kWave);
        lo1 = (uint32_t)__shfl((int)L.clo1, pos, kWave);
        lo2 = (uint32_t)__shfl((int)L.clo2, pos, kWave);
        L0 = (uint32_t)__shfl((int)L.cL0, pos, kWave);
        L1 = (uint32_t)__shfl((int)L.cL1, pos, kWave);
    }
    const uint32_t u = t - base;
    return u < L0 ? lo0 + u : (u < L0 + L1 ? lo1 + (u - L0) : lo2 + (u - L0 - L1));
}

// Sorted indices of the staging slots of a window of W candidates: slot k * 64 + lane holds
// stream position w0 + k * 64 + lane; positions past the stream repeat its last element.
template <int W = kWin>
__device__ __forceinline__ void window_indices(const LightStream& L, uint32_t w0, int lane,
                                               uint32_t j[W / kWave]) {
    static_assert(W % kWave == 0, "windows are whole rows of the wave");
#pragma unroll
    for (int k = 0; k < W / kWave; k++)
        j[k] = stream_index(L, min(w0 + (uint32_t)(k * kWave + lane), L.T - 1u));
}

// The lane's three row intervals clipped to the window [w0, w0 + W), as [jb[r], je[r]) with
// the longest first (three compare-swaps): a wave's r-th loop then runs as long as the longest
// r-th interval over its lanes, and lanes whose long row is not the same one share the first.
template <int W = kWin>
__device__ __forceinline__ void window_rows(const LightStream& L, uint32_t w0, uint32_t jb[3],
                                            uint32_t je[3]) {
#pragma unroll
    for (int r = 0; r < 3; r++) {
        jb[r] = max(L.S[r], w0);
        je[r] = max(min(L.S[r] + L.cnt[r], w0 + (uint32_t)W), jb[r]);
    }
    const auto cswap = [&](int a, int b) {
        const bool sw = je[b] - jb[b] > je[a] - jb[a];
        const uint32_t tb = jb[a], te = je[a];
        jb[a] = sw ? jb[b] : jb[a];
        je[a] = sw ? je[b] : je[a];
        jb[b] = sw ? tb : jb[b];
        je[b] = sw ? te : je[b];
    };
    cswap(0, 1);
    cswap(0, 2);
    cswap(1, 2);
}

}  // namespace fh
