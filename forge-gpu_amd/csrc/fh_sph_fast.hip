// fh_sph_fast.hip -- the fast SPH density and pressure/viscosity passes for gfx950.
//
// Work items.  Particles are processed in cell-sorted order.  An item is one (sub-tile, z-slab)
// pair: 64 consecutive sorted particles (one wavefront, one particle per lane) and one slab
// dz in {-1, 0, +1} of their 3x3x3 neighbourhood.  Each slab's partial sums go to a buffer of
// their own and k_prep / k_finalize add the three in a fixed order, so results are
// deterministic (no atomics) and a dense cell's work is split three ways.
//
// Light items (density_light, force_light: one wavefront per item).  For a fixed
// (dy, dz) the three x-adjacent cells of a particle are one contiguous range of the sorted
// arrays.  Lanes of one home row (cy, cz) are consecutive (a "segment"), and for each of the
// slab's three rows the union of a segment's ranges is again one contiguous range.  The wave
// concatenates the rows of all its segments into one candidate stream and copies it, kWin
// (256) candidates at a time, into its own LDS slice with coalesced 16-byte loads (no workgroup
// barrier); every lane then evaluates the intervals of its own rows that fall in the window
// (fh_stream.hpp, shared with the neighbour query of fh_grid.hip).  The plan builds each light
// item's stream once (the lanes' intervals and the first two windows' staging indices,
// kLightCacheWords) and both passes read it back; the few longer streams are rebuilt by each
// pass.  Light workgroups are renumbered so that runs of kXcdChunk consecutive items share one
// XCD's L2 (neighbouring sub-tiles read mostly the same cells).
//
// Heavy items.  An item whose particles face more than kHeavyWork (192) candidates in the slab,
// or that touches a co-located group, is listed by the plan (k_group_plan) and split into
// kHeavyWaves (4) parts: single-wave workgroups that hold the same 64 particles and take the
// 64-candidate chunks of each segment row round-robin (part p: chunks p, p + 4, ...).  Each part
// leaves its partial sums in hpart (by the item's list slot, hslot[item]), and k_prep /
// k_finalize add the parts in part order.  Heavy parts and light items share one launch per
// pass (k_density_pass, k_force_pass): the parts first, on workgroups 0 .. hparts - 1, the
// parts of an item on one XCD; light items after them.  (Two launches on two streams, a heavy
// kernel of 512-lane workgroups beside the light one, cost ~5 us of cross-queue wait at each
// fork and join.  8 parts per item were 2 % slower on c3 but 8 % faster on c4, whose dense clumps
// make long items; 2 or 16 parts 5 % and 8 % slower on c3.)
//
// Transposed items.  When an item's stream is many times longer than its largest particle's
// candidate count (sparse particles along a row beside a dense one), it is walked one particle
// at a time with the candidates across the lanes (coalesced loads, a wave reduction each).
//
// Co-located groups.  A cell of >= kCollapseMin (64) particles at one bitwise-identical point
// (c3's box corners collect thousands) is collapsed: the members are moved to the front of the
// cell, the first stands for all of them with weight M (and their summed velocity), and the
// others are finished from it in k_finalize with the viscosity weight of all three slabs.
//
// Arithmetic.  The reference's quantities (sph_density.rs:413-453, sph_fused.rs:552-637) with
// fused multiply-adds, the hardware reciprocal square root for 1/r, and per-particle force
// records (k_prep) that fold the constants in, so a pair costs one fma for its pressure factor;
// differences to the CPU restatement are rounding only (rel 1e-4 on density; 1e-4 of the sum of
// the pair terms' magnitudes, plus their float32 distance-rounding sensitivity, on
// accelerations).
#include "fh_internal.hpp"
#include "fh_stream.hpp"

namespace fh {

#ifndef FH_LW
#define FH_LW 1
#endif
// Light kernels: waves per workgroup.  One: a workgroup's LDS is released as soon as its item
// is done, however unequal the items (with several waves per workgroup the short items would
// hold LDS while the longest one runs).
constexpr int kLightWaves = FH_LW;
constexpr int kTileP = kLightWaves * 64;  // home particles per light workgroup
constexpr int kStage = 512;   // neighbour particles staged per chunk
constexpr uint32_t kEmpty = 0xFFFFFFFFu;

// p[i] if ok, else zero: the load always reads a valid element (index 0 when !ok) and the value
// is selected afterwards (a select between two addresses would compile to a FLAT load).
template <class T>
__device__ __forceinline__ T load_or(const T* __restrict__ p, uint32_t i, bool ok, T zero) {
    const T v = p[ok ? i : 0u];
    return ok ? v : zero;
}

// The three row ranges [b, e) of slab dz for one particle (cells clamped like the reference,
// sph_density.rs:421-437); empty ranges for rows outside the grid.
__device__ __forceinline__ void slab_ranges(const CellXYZ& c, bool live, const GridDesc& g,
                                            const uint32_t* __restrict__ cstart, uint32_t n,
                                            int dz, uint32_t b[3], uint32_t e[3]) {
#pragma unroll
    for (int r = 0; r < 3; r++) {
        b[r] = 0u;
        e[r] = 0u;
    }
    if (!live) return;
    const int cx = c.x, cy = c.y;
    const int nz = c.z + dz;
    if (nz < 0 || nz >= (int)g.nz) return;
    const uint32_t x0 = (uint32_t)(cx > 0 ? cx - 1 : 0);
    const uint32_t x1 = (uint32_t)(cx + 1 < (int)g.nx ? cx + 1 : (int)g.nx - 1);
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const int ny = cy + r - 1;
        if (ny < 0 || ny >= (int)g.ny) continue;
        const uint32_t row = (uint32_t)ny * g.nx + (uint32_t)nz * g.nx * g.ny;
        b[r] = cstart[row + x0];
        e[r] = min(cstart[row + x1 + 1u], n);
    }
}

// ---------------------------------------------------------------------------------------------
// Load balance.  A (64-particle sub-tile, slab) item whose particles each face more than
// kHeavyWork candidates -- the box corners of c3 collect thousands of particles at one point --
// is moved to a heavy list and processed in 4 single-wave parts that split the candidates of the
// same 64 particles; their partial sums are added in part order.  The light items skip those
// items.  The plan is made once per substep and serves both passes.
constexpr int kSub = 64;                // particles per sub-tile (one wavefront)
constexpr uint32_t kHeavyWork = 192;   // default: candidates per particle and slab
constexpr uint32_t kSmallHeavyWork = 32;  // the default below kSmallSystemN particles
constexpr uint32_t kCutFlag = 1u << 31;  // heavy list entry: the item touches a co-located group
constexpr uint32_t kTransFlag = 1u << 30;  // heavy list entry: walked transposed
constexpr uint32_t kEntryFlags = kCutFlag | kTransFlag;
// Item flags (the plan): light (one wavefront), heavy (heavy list), every particle co-located
// (skipped by both passes).
constexpr uint8_t kItemLight = 0, kItemHeavy = 1, kItemSkip = 2;
// hslot[item]: the heavy list slot of a heavy item (where its partial sums are), else kNoSlot.
constexpr uint32_t kNoSlot = 0xFFFFFFFFu;
// Partial-sum slot of the heavy entry at position pos of sub-list k: the lists interleaved, so a
// cap on the slots (FH_OPT_HEAVY_SLOTS) leaves every list its first entries.
__device__ __forceinline__ uint32_t heavy_slot(uint32_t k, uint32_t pos) {
    return pos * kHeavyLists + k;
}
// Transposed heavy items: the particles' candidate ranges overlap little (sparse particles
// spread along a row beside a dense one), so the union of a segment's ranges -- what the shared
// walk stages and every lane steps through -- is many times longer than any one particle's
// range.  The item is walked the other way round: one particle at a time, its candidates spread
// over the 64 lanes (coalesced loads), a wave reduction per particle.  Chosen for a heavy item
// when the stream is longer than kTransRatio times the largest particle's candidate count plus
// kTransOffset (below that the per-particle reductions cost more than the idle lanes), and for
// a light item only when it is pathologically longer (kTransLightRatio, kTransLightOffset): a
// light wave would then step through window after window serving one lane at a time.
#ifndef FH_TRANS_RATIO
#define FH_TRANS_RATIO 4
#endif
#ifndef FH_TRANS_LIGHT_RATIO
#define FH_TRANS_LIGHT_RATIO 16
#endif
#ifndef FH_TRANS_OFFSET
#define FH_TRANS_OFFSET 512
#endif
constexpr uint32_t kTransRatio = FH_TRANS_RATIO, kTransOffset = FH_TRANS_OFFSET;
constexpr uint32_t kTransLightRatio = FH_TRANS_LIGHT_RATIO, kTransLightOffset = 2048;
#ifndef FH_HGRID
#define FH_HGRID 4096
#endif
constexpr uint32_t kHeavyGrid = FH_HGRID;  // heavy workgroups (grid-stride over the list)
// candidates per step of the heavy force walk with chunk culling (twice as many without it,
// where the registers allow: the culling instantiation would spill)
#ifndef FH_HU
#define FH_HU 2
#endif

// Candidate density accumulation of one lane over [jb, je) of a staged chunk, four candidates
// per iteration with independent accumulators so LDS latency and the FMA chain overlap.
__device__ __forceinline__ float density_run(const float4* __restrict__ sp, uint32_t c0,
                                             uint32_t jb, uint32_t je, float4 pi, float h2,
                                             float acc) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    // pointer-stepped: one address and one compare per four candidates.  Callers may pass an
    // empty range with je < jb (a lane whose range ends before the chunk): the count is clamped
    // at 0, since je - c0 would wrap around.  The loop bounds are formed from the count, never
    // before the buffer: an address below the LDS buffer's start (at address 0 in the pass
    // kernels) would wrap around in 32-bit LDS addressing and the loop would run on for ~2^26
    // steps.
    const uint32_t m = je > jb ? je - jb : 0u;
    const float4* p = sp + (jb - c0);
    const float4* const pe = p + m;
    const float4* const pu = p + (m > 3u ? m - 3u : 0u);  // p < pu: four more candidates
    if (p < pu) {
        do {
            const float4 q0 = p[0], q1 = p[1], q2 = p[2], q3 = p[3];
            float dx = pi.x - q0.x, dy = pi.y - q0.y, dz = pi.z - q0.z;
            float d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
            a0 = fmaf(d * d, d, a0);
            dx = pi.x - q1.x; dy = pi.y - q1.y; dz = pi.z - q1.z;
            d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
            a1 = fmaf(d * d, d, a1);
            dx = pi.x - q2.x; dy = pi.y - q2.y; dz = pi.z - q2.z;
            d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
            a2 = fmaf(d * d, d, a2);
            dx = pi.x - q3.x; dy = pi.y - q3.y; dz = pi.z - q3.z;
            d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
            a3 = fmaf(d * d, d, a3);
            p += 4;
        } while (p < pu);
    }
    for (; p < pe; p++) {
        const float4 q = *p;
        const float dx = pi.x - q.x, dy = pi.y - q.y, dz = pi.z - q.z;
        const float d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
        a0 = fmaf(d * d, d, a0);
    }
    return acc + ((a0 + a1) + (a2 + a3));
}

// Co-located groups.  k_cell_starts lists the cells of >= kCollapseMin particles in which at
// least kGroupHits of kGroupSamples evenly spaced particles sit at the position of one of them.
// The group part of k_group_plan, one workgroup per listed cell, takes that sample's position
// P, counts the particles at exactly P (M) and,
// when M >= kCollapseMin, moves them to the front of the cell: the misplaced particles on both
// sides are ranked and swapped pairwise, in place.  The order inside such a cell then differs
// from ascending particle id (sums only change by rounding).
__device__ __forceinline__ bool same_pos(const float4& a, const float4& b) {
    return __float_as_uint(a.x) == __float_as_uint(b.x) &&
           __float_as_uint(a.y) == __float_as_uint(b.y) &&
           __float_as_uint(a.z) == __float_as_uint(b.z);
}

__device__ __forceinline__ void swap4(float4* p, uint32_t a, uint32_t b) {
    const float4 t = p[a];
    p[a] = p[b];
    p[b] = t;
}

constexpr int kGroupThreads = kPlanThreads;  // one launch: the same workgroup size
constexpr int kGroupWaves = kGroupThreads / kWave;
constexpr uint32_t kGroupUnroll = 8;  // particles loaded per thread before they are examined

// Workgroup sum of one value per thread, added in a fixed order (deterministic).
__device__ __forceinline__ float group_sum(float v, float* s_w) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int w = 0; w < kGroupWaves; w++) t += s_w[w];
    __syncthreads();
    return t;
}

// Bit k of the result: particle t + k (< t1) sits at P.  The loads are issued together from
// clamped indices.
__device__ __forceinline__ uint32_t match_bits(const float4* __restrict__ spos, uint32_t t,
                                               uint32_t t1, const float4& P) {
    float4 v[kGroupUnroll];
#pragma unroll
    for (uint32_t k = 0; k < kGroupUnroll; k++) v[k] = spos[min(t + k, t1 - 1u)];
    uint32_t m = 0;
#pragma unroll
    for (uint32_t k = 0; k < kGroupUnroll; k++)
        m |= (t + k < t1 && same_pos(v[k], P)) ? (1u << k) : 0u;
    return m;
}

// Blocked layout: thread t owns particles [f + t L, f + (t + 1) L) of the cell, L = ceil(cnt / 1024).
__device__ __forceinline__ void group_work(uint32_t bid, uint32_t nb, const uint2* __restrict__ big,
                                           uint32_t cap, uint32_t n,
                                           const uint32_t* __restrict__ skeys,
                                           const uint32_t* __restrict__ cstart,
                                           float4* __restrict__ spos, float4* __restrict__ svel,
                                           uint32_t* __restrict__ sidx,
                                           uint32_t* __restrict__ rank,
                                           uint32_t* __restrict__ scratch,
                                           uint64_t* __restrict__ cell_grp,
                                           float4* __restrict__ vrep,
                                           uint32_t* __restrict__ skip_tag,
                                           const Control* __restrict__ ctl) {
    __shared__ uint32_t s_scan[kGroupWaves];
    __shared__ float s_w[kGroupWaves];
    const uint32_t tid = threadIdx.x;
    const uint32_t count = min(ctl->big_count.v, cap);
    const uint32_t epoch = ctl->epoch;
    for (uint32_t q = bid; q < count; q += nb) {  // uniform
        const uint32_t f = big[q].x, cnt = min(cstart[skeys[f] + 1u], n) - f, end = f + cnt;
        const float4 P = spos[f + big[q].y];  // the sample that k_cell_starts matched
        const uint32_t L = ceil_div(cnt, (uint32_t)kGroupThreads);
        const uint32_t t0 = min(f + tid * L, end), t1 = min(t0 + L, end);
        // Membership bits of the thread's particles (L <= 32 kept in a register word; larger
        // cells are re-read in the later phases).
        const bool fits = L <= 32u;
        uint32_t bits = 0, mine = 0, M;
        for (uint32_t t = t0; t < t1; t += kGroupUnroll) {
            const uint32_t m = match_bits(spos, t, t1, P);
            mine += (uint32_t)__popc(m);
            if (fits) bits |= m << (t - t0);
        }
        (void)block_exclusive_scan<kGroupWaves>(mine, s_scan, &M);
        if (M < kCollapseMin) continue;  // uniform
        // misplaced particles: non-members before f + M, members from f + M on
        uint32_t nm = 0, mm = 0;
        for (uint32_t t = t0; t < t1; t += kGroupUnroll) {
            const uint32_t m = fits ? (bits >> (t - t0)) & 0xFFu : match_bits(spos, t, t1, P);
            for (uint32_t k = 0; k < kGroupUnroll && t + k < t1; k++) {
                const bool is = (m >> k) & 1u;
                if (t + k < f + M) nm += is ? 0u : 1u;
                else mm += is ? 1u : 0u;
            }
        }
        uint32_t tot;
        uint32_t knm = block_exclusive_scan<kGroupWaves>(nm, s_scan, &tot);
        uint32_t kmm = block_exclusive_scan<kGroupWaves>(mm, s_scan, &tot);
        // The misplaced slots in ascending order: the k-th non-member of [f, f + M) at
        // scratch[f + k], the k-th member of [f + M, end) at scratch[f + M + k] (k < tot <= M).
        for (uint32_t t = t0; t < t1; t += kGroupUnroll) {
            const uint32_t m = fits ? (bits >> (t - t0)) & 0xFFu : match_bits(spos, t, t1, P);
            for (uint32_t k = 0; k < kGroupUnroll && t + k < t1; k++) {
                const bool is = (m >> k) & 1u;
                if (t + k < f + M) {
                    if (!is) scratch[f + knm++] = t + k;
                } else if (is) {
                    scratch[f + M + kmm++] = t + k;
                }
            }
        }
        __threadfence_block();
        __syncthreads();
        // Thread k swaps the k-th misplaced member t with the k-th misplaced non-member u: all
        // pairs at once (their slots are distinct), so the cell costs one round of loads.
        for (uint32_t k = tid; k < tot; k += kGroupThreads) {
            const uint32_t t = scratch[f + M + k], u = scratch[f + k];
            // positions move, the .w index bits stay with the slot
            const float4 pt = spos[t], pu = spos[u];
            spos[t] = make_float4(pu.x, pu.y, pu.z, pt.w);
            spos[u] = make_float4(pt.x, pt.y, pt.z, pu.w);
            if (svel) swap4(svel, t, u);
            const uint32_t ti = sidx[t], ui = sidx[u];
            sidx[t] = ui;
            sidx[u] = ti;
            rank[ui] = t;
            rank[ti] = u;
        }
        __threadfence_block();
        __syncthreads();
        if (svel) {  // summed velocity of the group (fixed order)
            float vx = 0.0f, vy = 0.0f, vz = 0.0f;
            const uint32_t e1 = min(t1, f + M);
            for (uint32_t t = t0; t < e1; t += kGroupUnroll) {
                float4 v[kGroupUnroll];
#pragma unroll
                for (uint32_t k = 0; k < kGroupUnroll; k++) v[k] = svel[min(t + k, e1 - 1u)];
#pragma unroll
                for (uint32_t k = 0; k < kGroupUnroll; k++) {
                    if (t + k < e1) {
                        vx += v[k].x;
                        vy += v[k].y;
                        vz += v[k].z;
                    }
                }
            }
            vx = group_sum(vx, s_w);
            vy = group_sum(vy, s_w);
            vz = group_sum(vz, s_w);
            if (tid == 0) vrep[f] = make_float4(vx, vy, vz, 0.0f);
        }
        // tags in spos.w: the representative f carries kRepFlag | M, the other members f (the
        // positions moved above; the .w slot index bits stay with the slot)
        for (uint32_t t = f + tid; t < f + M; t += kGroupThreads)
            reinterpret_cast<float*>(spos + t)[3] = __uint_as_float(t == f ? (M | kRepFlag) : f);
        // sub-tiles made only of members are skipped by both passes (finished from f)
        for (uint32_t q = ceil_div(f + 1u, (uint32_t)kSub) + tid; (q + 1u) * kSub <= f + M;
             q += kGroupThreads)
            skip_tag[q] = epoch;
        if (tid == 0) cell_grp[skeys[f]] = ((uint64_t)epoch << 32) | M;
        __syncthreads();
    }
}

// Candidates of the possibly grouped cells among the 9 cells of a slab (tagged by
// k_cell_starts; the group part, which runs beside the plan, decides), as a count to subtract: such a
// cell of k particles is counted as one (a group of M counts as one candidate, M <= k).
__device__ __forceinline__ uint32_t grouped_excess(const CellXYZ& hc, const GridDesc& g,
                                                   const uint64_t* __restrict__ cand_tag,
                                                   const uint32_t* __restrict__ cstart,
                                                   uint32_t epoch, int dz) {
    const int cx = hc.x, cy = hc.y, cz = hc.z + dz;
    if (cz < 0 || cz >= (int)g.nz) return 0u;
    uint32_t ex = 0;
    for (int y = cy - 1; y <= cy + 1; y++) {
        if (y < 0 || y >= (int)g.ny) continue;
        for (int x = cx - 1; x <= cx + 1; x++) {
            if (x < 0 || x >= (int)g.nx) continue;
            const uint32_t c = (uint32_t)x + (uint32_t)y * g.nx + (uint32_t)cz * g.nx * g.ny;
            if ((uint32_t)(cand_tag[c] >> 32) == epoch) ex += cstart[c + 1u] - cstart[c] - 1u;
        }
    }
    return ex;
}

// Weight of a candidate from its spos.w bits: 1 for an ordinary particle, M for a group
// representative, 0 for the other members of a group (they are counted by the representative).
__device__ __forceinline__ float candidate_weight(float wbits, uint32_t j) {
    const uint32_t w = __float_as_uint(wbits);
    if (w & kRepFlag) return (float)(w & ~kRepFlag);
    return w == j ? 1.0f : 0.0f;
}

// density_run over candidates staged with their weight in .w (heavy kernels: groups staged
// in full, members with weight 0).
__device__ __forceinline__ float density_run_w(const float4* __restrict__ sp, uint32_t c0,
                                               uint32_t jb, uint32_t je, float4 pi, float h2,
                                               float acc) {
    float a0 = 0.0f, a1 = 0.0f;
    const uint32_t m = je > jb ? je - jb : 0u;  // empty when je <= jb
    const float4* p = sp + (jb - c0);
    const float4* const pe = p + m;
    const float4* const pu = p + (m > 1u ? m - 1u : 0u);  // p < pu: two more (as density_run)
    if (p < pu) {
        do {
            const float4 q0 = p[0], q1 = p[1];
            float dx = pi.x - q0.x, dy = pi.y - q0.y, dz = pi.z - q0.z;
            float d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
            a0 = fmaf(q0.w * d, d * d, a0);
            dx = pi.x - q1.x; dy = pi.y - q1.y; dz = pi.z - q1.z;
            d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
            a1 = fmaf(q1.w * d, d * d, a1);
            p += 2;
        } while (p < pu);
    }
    if (p < pe) {
        const float4 q = *p;
        const float dx = pi.x - q.x, dy = pi.y - q.y, dz = pi.z - q.z;
        const float d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
        a0 = fmaf(q.w * d, d * d, a0);
    }
    return acc + (a0 + a1);
}

__device__ __forceinline__ uint32_t pick3(const uint32_t v[3], int r) {
    return r == 0 ? v[0] : (r == 1 ? v[1] : v[2]);
}

// Home-row segments.  A wave owns 64 consecutive sorted particles (a sub-tile); the particles of
// one home row (cy, cz) are consecutive lanes, and for each of the slab's 3 rows the union of
// their neighbour ranges is one contiguous range (x-adjacent cells of that row only): from the
// first lane's begin to the last lane's end.
__device__ __forceinline__ uint32_t home_row(const CellXYZ& c, const GridDesc& g) {
    return (uint32_t)c.y + (uint32_t)c.z * g.ny;
}

// Length of the wave's candidate stream for one slab (the sum over home-row segments of the
// unions of their rows, as laid out by light_stream).
__device__ __forceinline__ uint32_t stream_total(const uint32_t b[3], const uint32_t e[3],
                                                 uint32_t hr, bool in, int lane) {
    const uint32_t hnext = (uint32_t)__shfl_down((int)hr, 1u, kWave);
    const bool innext = __shfl_down((int)in, 1u, kWave) != 0 && lane < 63;
    const uint32_t hprev = (uint32_t)__shfl_up((int)hr, 1u, kWave);
    const uint64_t starts = __ballot(in && (lane == 0 || hprev != hr));
    const bool last = in && !(innext && hnext == hr);
    // the leader's begins, read by the segment's last lane
    const uint64_t upto = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
    const uint64_t before = starts & upto;
    const int leader = before ? 63 - __clzll((long long)before) : 0;
    uint32_t len = 0;
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const uint32_t lo = (uint32_t)__shfl((int)b[r], leader, kWave);
        len += last ? e[r] - lo : 0u;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) len += (uint32_t)__shfl_xor((int)len, off, kWave);
    return len;
}

// A member of a co-located group other than its representative (spos.w bits of sorted slot j).
__device__ __forceinline__ bool is_member(uint32_t bits, uint32_t j) {
    return !(bits & kRepFlag) && bits != j;
}

// Lanes w, w + hw, w + 2 hw, ... of a wave (the particles wave w takes in a transposed walk).
__device__ __forceinline__ uint64_t trans_lanes(int wave, int hw) {
    uint64_t m = 0;
    for (int l = wave; l < kWave; l += hw) m |= 1ull << l;
    return m;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Next chunk start of a transposed walk: j0 + 64, or past a co-located group whose
// representative (spos.w = kRepFlag | M) is in this chunk and whose members run beyond it.
__device__ __forceinline__ uint32_t trans_next(uint32_t j0, uint32_t j, bool ok, uint32_t wb) {
    const bool rep = ok && (wb & kRepFlag);
    uint32_t nx = j0 + (uint32_t)kWave;
    if (__ballot(rep) != 0ull) nx = max(nx, wave_max(rep ? j + (wb & ~kRepFlag) : 0u));
    return nx;
}

// Transposed density walk of the item's particles taken by this wave: returns, in the lane of
// each such particle, its density partial (sum of w (h^2 - r^2)^3; weights from spos.w).
__device__ __forceinline__ float density_trans(const float4* __restrict__ spos,
                                               const uint32_t b[3], const uint32_t e[3],
                                               const float4& pi, bool mine, float h2,
                                               uint64_t lanes, int lane) {
    float out = 0.0f;
    uint64_t todo = __ballot(mine) & lanes;
    while (todo) {  // uniform
        const int l = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1ull;
        const float px = __shfl(pi.x, l, kWave), py = __shfl(pi.y, l, kWave),
                    pz = __shfl(pi.z, l, kWave);
        float acc = 0.0f;
#pragma unroll
        for (int r = 0; r < 3; r++) {
            const uint32_t bb = (uint32_t)__shfl((int)b[r], l, kWave);
            const uint32_t ee = (uint32_t)__shfl((int)e[r], l, kWave);
            for (uint32_t j0 = bb; j0 < ee;) {  // uniform
                const uint32_t j = j0 + (uint32_t)lane;
                const bool ok = j < ee;
                const float4 q = spos[ok ? j : j0];
                const uint32_t wb = __float_as_uint(q.w);
                const float c = ok ? ((wb & kRepFlag) ? (float)(wb & ~kRepFlag)
                                                      : (wb == j ? 1.0f : 0.0f))
                                   : 0.0f;
                const float dx = px - q.x, dy = py - q.y, dz = pz - q.z;
                const float d = fmaxf(fmaf(-dz, dz, fmaf(-dy, dy, fmaf(-dx, dx, h2))), 0.0f);
                acc = fmaf(c * d, d * d, acc);
                j0 = trans_next(j0, j, ok, wb);
            }
        }
        acc = wave_sum(acc);
        if (lane == l) out = acc;
    }
    return out;
}

// Below this many particles the plan leaves the light streams to the density pass: the
// plan's waves then run in one round, so the stream build would lengthen it one for one.
constexpr uint32_t kPlanStreamMinN = 1u << 18;

// Base of a light item's kept stream in slab dz: a sorted index at or below every index of the
// stream, when every index lies within 65,536 slots of it (the kept stream holds 16-bit offsets
// from it; an empty stream keeps with base 0), else kNoBase: the stream is not kept.  Every
// candidate cell of a particle in cell id lies in [id - 1 - nx + nx ny dz, id + 1 + nx + nx ny dz]
// (linear ids x + nx (y + ny z)) and the item's particles are sorted by cell id, so the cell
// starts at its first particle's low end and past its last particle's high end (stream_bounds,
// loaded beside the slab's ranges) bound the stream (the gaps a stream holds between lanes'
// ranges lie inside those ranges' span).  Wave-uniform; call with the whole wave (the lanes in
// the tile lead).
constexpr uint32_t kNoBase = 0xFFFFFFFFu;
__device__ __forceinline__ uint2 stream_bounds(uint32_t key, bool in, const GridDesc& g,
                                               const uint32_t* __restrict__ cstart, int dz) {
    const int last = __popcll(__ballot(in)) - 1;
    const int64_t plane = (int64_t)g.nx * g.ny, cells = plane * g.nz;
    const int64_t k0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)key);
    const int64_t k1 = (uint32_t)__builtin_amdgcn_readlane((int)key, last);
    const int64_t lo = k0 - 1 - (int64_t)g.nx + plane * dz;
    const int64_t hi = k1 + 2 + (int64_t)g.nx + plane * dz;
    return make_uint2(cstart[min(max(lo, (int64_t)0), cells)],
                      cstart[min(max(hi, (int64_t)0), cells)]);
}
__device__ __forceinline__ uint32_t stream_base(uint2 bounds, uint32_t T) {
    if (T == 0u) return 0u;
    return bounds.y - bounds.x <= 65536u ? bounds.x : kNoBase;
}

// A kept stream's lane intervals: a kept stream has at most 2 kWin = 512 positions, so each
// lane's three starts and three counts fit 10 bits each, in two words (lane l: words l and
// 64 + l; the starts of lanes outside the tile, whose counts are 0, are masked).  The window
// offsets follow (kLightHead words in).
constexpr uint32_t kLightHead = 2 * kWave;
static_assert(2 * kWin < 1024, "kept stream positions fit 10 bits");
__device__ __forceinline__ void put_intervals(uint32_t* __restrict__ lc, int lane,
                                              const LightStream& L) {
    lc[lane] = (L.S[0] & 0x3FFu) | (L.S[1] & 0x3FFu) << 10 | (L.S[2] & 0x3FFu) << 20;
    lc[kWave + lane] = L.cnt[0] | L.cnt[1] << 10 | L.cnt[2] << 20;
}
__device__ __forceinline__ void get_intervals(const uint32_t* __restrict__ lc, int lane,
                                              LightStream& L) {
    const uint32_t s = lc[lane], c = lc[kWave + lane];
#pragma unroll
    for (int r = 0; r < 3; r++) {
        L.S[r] = (s >> (10 * r)) & 0x3FFu;
        L.cnt[r] = (c >> (10 * r)) & 0x3FFu;
    }
}

// A kept window's staging indices as 16-bit offsets from the base, two per word: lane l's words
// of the window at w0 hold slots (l, 64 + l) and (128 + l, 192 + l).
static_assert(kWinLoads % 2 == 0, "window slots pair up");
__device__ __forceinline__ void put_offsets(uint32_t* __restrict__ off, uint32_t w0, int lane,
                                            const uint32_t j[kWinLoads], uint32_t base) {
#pragma unroll
    for (int k = 0; k < kWinLoads; k += 2)
        off[w0 / 2u + (uint32_t)(k / 2 * kWave + lane)] = (j[k] - base) | ((j[k + 1] - base) << 16);
}
__device__ __forceinline__ void get_offsets(const uint32_t* __restrict__ off, uint32_t w0,
                                            int lane, uint32_t j[kWinLoads], uint32_t base) {
#pragma unroll
    for (int k = 0; k < kWinLoads; k += 2) {
        const uint32_t v = off[w0 / 2u + (uint32_t)(k / 2 * kWave + lane)];
        j[k] = base + (v & 0xFFFFu);
        j[k + 1] = base + (v >> 16);
    }
}

// Plan, beside the co-located groups (the group part, which tags particles f+1 .. f+M-1 of a grouped
// cell in spos[s].w with their representative f, f itself with kRepFlag | M, and marks the
// sub-tiles made only of such non-representative particles in skip_tag: both passes skip them,
// their particles take the representative's density, and its acceleration up to the viscosity
// term that depends on the particle's own velocity, in k_finalize).  A (sub-tile, slab) item is
// heavy when its largest per-particle candidate count (a cell that may hold a group counting
// once) exceeds heavy_work or when it touches such a cell, and transposed (heavy) when its
// stream is much longer than that count.
__device__ __forceinline__ void plan_work(uint32_t bid, const uint32_t* __restrict__ skeys,
                                          uint32_t n, GridDesc g,
                                          const uint32_t* __restrict__ cstart,
                                          const uint64_t* __restrict__ cand_tag,
                                          uint8_t* __restrict__ flag,
                                          uint32_t* __restrict__ heavy, uint32_t heavy_cap,
                                          uint32_t heavy_work, uint32_t direct_mode,
                                          Control* ctl, uint32_t* __restrict__ lstream,
                                          uint2* __restrict__ lstream_t,
                                          uint32_t* __restrict__ hslot, uint32_t hslot_cap) {
    constexpr int kWaves = kPlanThreads / kWave;
    __shared__ uint32_t s_item[kWaves * 3];
    __shared__ uint32_t s_count[kWaves];
    const uint32_t s = bid * blockDim.x + threadIdx.x;
    const uint32_t sub = s / kSub;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool live = s < n;
    uint32_t nh = 0;  // heavy items of this wave, kept in s_item[wave * 3 ...]
    if (sub * kSub < n) {  // wave-uniform
        const uint32_t key = load_or(skeys, s, live, 0u);
        const CellXYZ ci = key_xyz(key, g);
        {
            const uint32_t epoch = ctl->epoch;
            for (int slab = 0; slab < 3; slab++) {
                uint32_t b[3], e[3];
                slab_ranges(ci, live, g, cstart, n, slab - 1, b, e);
                const uint2 bounds = stream_bounds(key, live, g, cstart, slab - 1);
                uint32_t cand = (e[0] - b[0]) + (e[1] - b[1]) + (e[2] - b[2]);
                uint32_t excess = 0;
                if (cand >= kCollapseMin) {  // a grouped cell holds at least kCollapseMin
                    excess = grouped_excess(ci, g, cand_tag, cstart, epoch, slab - 1);
                    cand -= excess;
                }
                const uint32_t w = wave_max(cand);
                const bool touches = __ballot(excess > 0u) != 0ull;
                bool hv = w > heavy_work || touches;  // light items hold no group
                bool trans = direct_mode == 2u;
                LightStream L;
                L.T = ~0u;  // no stream built
                if (direct_mode == 1u) {
                    // a light item only when its stream is far longer (pathologically
                    // disjoint ranges: one window would serve one lane at a time); the stream
                    // of a light candidate is built in full, for the passes to reuse
                    const bool build = !hv && n >= kPlanStreamMinN;  // uniform
                    if (build) light_stream(L, b, e, home_row(ci, g), live, lane);
                    const uint32_t T = build ? L.T : stream_total(b, e, home_row(ci, g), live, lane);
                    trans = hv ? T > kTransRatio * w + kTransOffset
                               : T > kTransLightRatio * w + kTransLightOffset;
                }
                hv = hv || trans;
                const uint32_t item = sub * 3u + (uint32_t)slab;
                // uniform: the light stream for both passes (L.T is ~0u when none was built)
                const uint32_t base =
                    !hv && L.T <= 2u * kWin ? stream_base(bounds, L.T) : kNoBase;
                if (base != kNoBase) {
                    uint32_t* lc = lstream + (size_t)item * kLightCacheWords;
                    put_intervals(lc, lane, L);
                    for (uint32_t w0 = 0; w0 < L.T; w0 += kWin) {  // uniform
                        uint32_t j[kWinLoads];
                        window_indices(L, w0, lane, j);
                        put_offsets(lc + kLightHead, w0, lane, j, base);
                    }
                }
                if (lane == 0) {
                    lstream_t[item] = make_uint2(hv ? ~0u : L.T, base);
                    flag[item] = hv ? kItemHeavy : kItemLight;
                    if (!hv) hslot[item] = kNoSlot;
                    if (hv)
                        s_item[wave * 3 + (int)nh] =
                            item | (touches ? kCutFlag : 0u) | (trans ? kTransFlag : 0u);
                }
                nh += hv ? 1u : 0u;
            }
        }
    }
    if (lane == 0) s_count[wave] = nh;
    __syncthreads();
    // one append per workgroup, to sub-list blockIdx % kHeavyLists, in wave order; the entry
    // at position pos of list k has partial-sum slot heavy_slot(k, pos) if that is below
    // hslot_cap, else none (kNoSlot: the passes' part-0 wave walks every part of it)
    __shared__ uint32_t s_base;
    if (threadIdx.x == 0) {
        uint32_t tot = 0;
        for (int w = 0; w < kWaves; w++) tot += s_count[w];
        s_base = tot ? atomicAdd(&ctl->heavy_count[bid % kHeavyLists].v, tot) : 0u;
    }
    __syncthreads();
    if (threadIdx.x < kWaves * 3) {
        const int w = threadIdx.x / 3, k = threadIdx.x - 3 * (threadIdx.x / 3);
        uint32_t off = 0;
        for (int v = 0; v < w; v++) off += s_count[v];
        if ((uint32_t)k < s_count[w]) {
            const uint32_t pos = s_base + off + (uint32_t)k;
            const uint32_t ent = s_item[w * 3 + k];
            const uint32_t slot = heavy_slot(bid % kHeavyLists, pos);
            // the sub-lists hold every item of the context (heavy_cap): pos < heavy_cap always
            if (pos < heavy_cap) heavy[(bid % kHeavyLists) * heavy_cap + pos] = ent;
            hslot[ent & ~kEntryFlags] = pos < heavy_cap && slot < hslot_cap ? slot : kNoSlot;
        }
    }
}

// Co-located groups and the work plan in one launch: the first kGroupBlocks workgroups walk the
// candidate group cells (k_cell_starts' list), the others plan the items.  The plan needs only
// the cells that may hold a group (tagged by k_cell_starts), not their outcome, and every
// particle of a cell gives the cell's neighbour ranges whether or not it has been moved yet.
constexpr uint32_t kGroupBlocks = 64;
// 8 waves per SIMD (64 registers, a few spilled): the plan mostly waits on its cell-range loads
// and the shuffles of the stream build, so occupancy pays more than the registers.
__global__ __launch_bounds__(kPlanThreads, 8) void k_group_plan(
    const uint2* __restrict__ big, uint32_t cap, uint32_t n, const uint32_t* __restrict__ skeys,
    const uint32_t* __restrict__ cstart, float4* __restrict__ spos, float4* __restrict__ svel,
    uint32_t* __restrict__ sidx, uint32_t* __restrict__ rank, uint32_t* __restrict__ scratch,
    uint64_t* __restrict__ cell_grp, float4* __restrict__ vrep, uint32_t* __restrict__ skip_tag,
    GridDesc g, const uint64_t* __restrict__ cand_tag, uint8_t* __restrict__ flag,
    uint32_t* __restrict__ heavy, uint32_t heavy_cap, uint32_t heavy_work, uint32_t direct_mode,
    Control* ctl, uint32_t* __restrict__ lstream, uint2* __restrict__ lstream_t,
    uint32_t* __restrict__ hslot, uint32_t hslot_cap) {
    if (blockIdx.x < kGroupBlocks)
        group_work(blockIdx.x, kGroupBlocks, big, cap, n, skeys, cstart, spos, svel, sidx, rank,
                   scratch, cell_grp, vrep, skip_tag, ctl);
    else
        plan_work(blockIdx.x - kGroupBlocks, skeys, n, g, cstart, cand_tag, flag, heavy,
                  heavy_cap, heavy_work, direct_mode, ctl, lstream, lstream_t, hslot, hslot_cap);
}

// The heavy work lists of this substep as one sequence: entry q of the concatenation of the
// kHeavyLists sub-lists.  heavy_total() is their total length.
__device__ __forceinline__ uint32_t heavy_total(const Control* __restrict__ ctl, uint32_t cap) {
    uint32_t t = 0;
#pragma unroll
    for (int q = 0; q < kHeavyLists; q++) t += min(ctl->heavy_count[q].v, cap);
    return t;
}

// ---------------------------------------------------------------------------------------------
// Lane `lane` of a chunk of m (>= 1) candidates starting at c0: a global load from a clamped,
// always valid index, zeroed past the chunk.  (A conditional load written as `lane < m ?
// spos[c0 + lane] : zero` selects between two addresses and compiles to a FLAT load, which
// also counts against the LDS wait counter and so serialises with the LDS staging.)
__device__ __forceinline__ float4 chunk_load(const float4* __restrict__ spos, uint32_t c0,
                                             uint32_t m, int lane) {
    const float4 v = spos[c0 + min((uint32_t)lane, m - 1u)];
    return (uint32_t)lane < m ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// Bounding box of the positions of the lanes with `on` (uniform; no such lane: lo = +inf,
// hi = -inf, which no candidate is near).  NaN coordinates are ignored (fminf / fmaxf); a lane
// whose coordinate is NaN has no pair at all.
struct Box {
    float lx, ly, lz, hx, hy, hz;
};
// (the reduced value is the same in every lane: read from lane 0 into a scalar register)
__device__ __forceinline__ float wave_fmin(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fminf(v, __shfl_xor(v, o, kWave));
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ float wave_fmax(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ Box lane_box(const float4& p, bool on) {
    const float inf = __builtin_inff();
    Box b;
    b.lx = wave_fmin(on ? p.x : inf);
    b.ly = wave_fmin(on ? p.y : inf);
    b.lz = wave_fmin(on ? p.z : inf);
    b.hx = wave_fmax(on ? p.x : -inf);
    b.hy = wave_fmax(on ? p.y : -inf);
    b.hz = wave_fmax(on ? p.z : -inf);
    return b;
}

// The lanes whose candidate of a chunk (this lane's v, if `valid`) lies within sqrt(lim) of
// the box (a chunk with none is skipped).  The distance of a pair is at least its candidate's distance to the box of the other
// particles, so a chunk with no candidate within h of the item's box holds no pair of its
// particles; lim = h^2 (1 + 2^-10) leaves room for the rounding of either computation.  A NaN
// candidate coordinate counts as near (the pair test rejects it).
__device__ __forceinline__ uint64_t near_mask(const float4& v, bool valid, const Box& b,
                                              float lim) {
    const float dx = fmaxf(fmaxf(b.lx - v.x, v.x - b.hx), 0.0f);
    const float dy = fmaxf(fmaxf(b.ly - v.y, v.y - b.hy), 0.0f);
    const float dz = fmaxf(fmaxf(b.lz - v.z, v.z - b.hz), 0.0f);
    return __ballot(valid && fmaf(dz, dz, fmaf(dy, dy, dx * dx)) <= lim);
}

// Rows (bit r) whose interval [b[r], e[r]) is the same in every lane of the segment: each chunk
// of such a row lies inside every lane's interval, so it can be compacted to its candidates near
// the item's box (near_mask) before the pair loop.
__device__ __forceinline__ uint32_t same_rows(const uint32_t b[3], const uint32_t e[3], bool mine,
                                              int leader) {
    uint32_t same = 0u;
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)b[r], leader);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)e[r], leader);
        if (__ballot(mine && (b[r] != lo || e[r] != hi)) == 0ull) same |= 1u << r;
    }
    return same;
}

// Position of this lane among the set bits of `mask` below it.
__device__ __forceinline__ uint32_t mask_rank(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Next non-empty row after r (3 if none) of a segment whose row r spans [lo[r], hi[r]).
__device__ __forceinline__ int next_row(const uint32_t lo[3], const uint32_t hi[3], int r) {
    for (r = r + 1; r < 3; r++)
        if (pick3(lo, r) < pick3(hi, r)) break;
    return r;
}

static_assert(kLightCacheWords == kLightHead + kWin, "light stream cache layout");

// Density partials: dpart[slab][s] = sum over the slab's neighbours j of (h^2 - r^2)^3, r^2 < h^2.
// Light items hold no co-located group (the plan sends those to the heavy list).
__device__ __forceinline__ void density_light(uint32_t item, int lane, float4* buf,
                                              const float4* __restrict__ spos,
                                              const uint32_t* __restrict__ skeys, uint32_t n,
                                              GridDesc g, const uint32_t* __restrict__ cstart,
                                              float h2, float* __restrict__ dpart,
                                              uint32_t stride, uint32_t items,
                                              const uint8_t* __restrict__ flag,
                                              const uint32_t* __restrict__ skip_tag,
                                              const Control* __restrict__ ctl,
                                              uint32_t* __restrict__ lstream,
                                              uint2* __restrict__ lstream_t) {
    if (item >= items || flag[item] != kItemLight) return;  // whole wave
    const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
    if (skip_tag[sub] == ctl->epoch) return;  // only group members (finished from the group)
    const uint32_t s = sub * kSub + (uint32_t)lane;
    const bool in = s < n;
    const float4 pi = load_or(spos, s, in, make_float4(0.0f, 0.0f, 0.0f, 0.0f));
    // the candidate stream the plan built (short streams), else built here and, when short,
    // kept for the force pass (kLightCacheWords)
    LightStream L;
    const uint2 tb = lstream_t[item];
    L.T = tb.x;
    uint32_t base = tb.y;
    const bool kept = base != kNoBase;  // uniform
    bool keep = false;
    uint32_t* lc = lstream + (size_t)item * kLightCacheWords;
    if (kept) {
        get_intervals(lc, lane, L);
    } else {
        const uint32_t key = load_or(skeys, s, in, 0u);
        const CellXYZ ci = key_xyz(key, g);
        uint32_t b[3], e[3];
        slab_ranges(ci, in, g, cstart, n, (int)slab - 1, b, e);
        const uint2 bounds = stream_bounds(key, in, g, cstart, (int)slab - 1);
        light_stream(L, b, e, home_row(ci, g), in, lane);
        base = L.T <= 2u * kWin ? stream_base(bounds, L.T) : kNoBase;  // uniform
        keep = base != kNoBase;
        if (lane == 0) lstream_t[item] = make_uint2(L.T, base);
        if (keep) {
            put_intervals(lc, lane, L);
        }
    }
    float acc = 0.0f;
    for (uint32_t w0 = 0; w0 < L.T; w0 += kWin) {  // wave-uniform
        uint32_t j[kWinLoads];
        if (kept) {
            get_offsets(lc + kLightHead, w0, lane, j, base);
        } else {
            window_indices(L, w0, lane, j);
            if (keep) put_offsets(lc + kLightHead, w0, lane, j, base);
        }
        float4 v[kWinLoads];
#pragma unroll
        for (int k = 0; k < kWinLoads; k++) v[k] = spos[j[k]];
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < kWinLoads; k++) buf[k * kWave + lane] = v[k];
        __builtin_amdgcn_wave_barrier();
        uint32_t jb[3], je[3];
        window_rows(L, w0, jb, je);
#pragma unroll
        for (int r = 0; r < 3; r++)
            if (jb[r] < je[r]) acc = density_run(buf, w0, jb[r], je[r], pi, h2, acc);
    }
    if (in) dpart[(size_t)slab * stride + s] = acc;
}

// Heavy items: the parts of an item (single-wave workgroups) hold the same 64 particles of one
// (sub-tile, slab) and walk the same home-row segments as density_light, but split each segment
// row's chunks round-robin (part w takes chunks w, w + 4, ...), each through its own LDS; their
// partial sums are added in part order by the passes' consumers.  The members of co-located
// groups in a segment row are cut out of its candidate range (the representative stays, with
// weight M).
constexpr int kMaxCut = 4;  // groups cut out per segment row (further ones are staged, weight 0)

struct RowPlan {
    uint32_t lo[kMaxCut + 1], hi[kMaxCut + 1];
    uint32_t k, total;  // sub-ranges, chunks
};

// Sub-ranges of one segment row [lo, hi), which covers cells xa..xb of the row at rowbase.
__device__ __forceinline__ void row_plan(RowPlan& R, uint32_t lo, uint32_t hi, uint32_t rowbase,
                                         int xa, int xb, const uint32_t* __restrict__ cstart,
                                         const uint64_t* __restrict__ cell_grp, uint32_t epoch,
                                         int lane) {
    R.k = 0;
    uint32_t cur = lo;
    for (int x0 = xa; x0 <= xb; x0 += kWave) {  // uniform
        const int x = x0 + lane;
        bool grp = false;
        uint32_t f = 0, M = 0;
        if (x <= xb) {
            const uint64_t gv = cell_grp[rowbase + (uint32_t)x];
            if ((uint32_t)(gv >> 32) == epoch) {
                grp = true;
                M = (uint32_t)gv;
                f = cstart[rowbase + (uint32_t)x];
            }
        }
        uint64_t bal = __ballot(grp);
        while (bal) {  // uniform
            const int l = __ffsll((unsigned long long)bal) - 1;
            bal &= bal - 1ull;
            const uint32_t fl = (uint32_t)__builtin_amdgcn_readlane((int)f, l);
            const uint32_t ml = (uint32_t)__builtin_amdgcn_readlane((int)M, l);
            if (R.k < (uint32_t)kMaxCut) {
#pragma unroll
                for (int i = 0; i < kMaxCut; i++)
                    if ((uint32_t)i == R.k) {
                        R.lo[i] = cur;
                        R.hi[i] = fl + 1u;
                    }
                R.k++;
                cur = fl + ml;
            }
        }
    }
#pragma unroll
    for (int i = 0; i <= kMaxCut; i++)
        if ((uint32_t)i == R.k) {
            R.lo[i] = cur;
            R.hi[i] = hi;
        }
    R.k++;
    R.total = 0;
#pragma unroll
    for (int i = 0; i <= kMaxCut; i++)
        if ((uint32_t)i < R.k) R.total += (R.hi[i] - R.lo[i] + kWave - 1) / kWave;
}

__device__ __forceinline__ void row_chunk(const RowPlan& R, uint32_t q, uint32_t& c0,
                                          uint32_t& m) {
    c0 = 0;
    m = 0;
#pragma unroll
    for (int i = 0; i <= kMaxCut; i++) {
        if ((uint32_t)i < R.k && m == 0) {
            const uint32_t nc = (R.hi[i] - R.lo[i] + kWave - 1) / kWave;
            if (q < nc) {
                c0 = R.lo[i] + q * kWave;
                m = min((uint32_t)kWave, R.hi[i] - c0);
            } else {
                q -= nc;
            }
        }
    }
}

// Cells xa..xb and base index of row r of slab dz for a lane in cell c (valid = row inside the
// grid).
__device__ __forceinline__ bool seg_row(const CellXYZ& c, const GridDesc& g, int dz, int r,
                                        uint32_t& rowbase, int& cx) {
    cx = c.x;
    const int cy = c.y + r - 1;
    const int cz = c.z + dz;
    rowbase = (uint32_t)cy * g.nx + (uint32_t)cz * g.nx * g.ny;
    return cy >= 0 && cy < (int)g.ny && cz >= 0 && cz < (int)g.nz;
}

// Chunk t of a segment whose rows r = 0..2 have the plans R[r] (rows in order): row, first
// candidate and size; r = 3 past the end.
__device__ __forceinline__ void seg_chunk(const RowPlan R[3], uint32_t t, int& r, uint32_t& c0,
                                          uint32_t& m) {
    r = 3;
    c0 = 0;
    m = 0;
    if (t < R[0].total) {
        r = 0;
    } else if (t < R[0].total + R[1].total) {
        r = 1;
        t -= R[0].total;
    } else if (t < R[0].total + R[1].total + R[2].total) {
        r = 2;
        t -= R[0].total + R[1].total;
    } else {
        return;
    }
    if (r == 0) row_chunk(R[0], t, c0, m);  // constant indices: the plans stay in registers
    else if (r == 1) row_chunk(R[1], t, c0, m);
    else row_chunk(R[2], t, c0, m);
}

// The plans of the 3 rows of a segment (leader / last lane of the segment): the row union,
// cut around co-located groups when the item touches any (`cut`).
__device__ __forceinline__ void seg_plans(RowPlan R[3], const CellXYZ& ci, const GridDesc& g,
                                          int dz, const uint32_t b[3], const uint32_t e[3],
                                          int leader, int last, bool cut,
                                          const uint32_t* __restrict__ cstart,
                                          const uint64_t* __restrict__ cell_grp, uint32_t epoch,
                                          int lane) {
#pragma unroll
    for (int r = 0; r < 3; r++) {
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)b[r], leader);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)e[r], last);
        R[r].k = 1;
        R[r].lo[0] = lo;
        R[r].hi[0] = lo < hi ? hi : lo;
        R[r].total = lo < hi ? (hi - lo + kWave - 1) / kWave : 0u;
        if (cut && lo < hi) {
            uint32_t rowbase;
            int cx;
            (void)seg_row(ci, g, dz, r, rowbase, cx);
            rowbase = (uint32_t)__builtin_amdgcn_readlane((int)rowbase, leader);
            const int xa = max(__builtin_amdgcn_readlane(cx, leader) - 1, 0);
            const int xb = min(__builtin_amdgcn_readlane(cx, last) + 1, (int)g.nx - 1);
            row_plan(R[r], lo, hi, rowbase, xa, xb, cstart, cell_grp, epoch, lane);
        }
    }
}


// One virtual wave (`wave` of hw) of heavy entry `entry`: its partial density sums (chunks
// wave, wave + hw, ... of each segment row; the transposed walk's lanes trans_lanes(wave, hw)),
// hw = the item's part count.
// False when the item is skipped (only group members).
template <bool CULL>
__device__ __forceinline__ bool density_heavy_wave(
    uint32_t entry, int wave, int hw, int lane, float4* buf, const float4* __restrict__ spos,
    const uint32_t* __restrict__ skeys, uint32_t n, GridDesc g,
    const uint32_t* __restrict__ cstart, const uint64_t* __restrict__ cell_grp, float h2,
    const uint32_t* __restrict__ skip_tag, uint32_t epoch, float& out) {
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const bool cut = (entry & kCutFlag) != 0u;  // the item touches a co-located group
    const bool trans = (entry & kTransFlag) != 0u;
    const uint32_t item = entry & ~kEntryFlags;
    const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
    if (skip_tag[sub] == epoch) return false;  // uniform: only group members
    const uint32_t s = sub * kSub + (uint32_t)lane;
    const bool live = s < n;
    const float4 pi = load_or(spos, s, live, z4);
    // the item's box, for skipping chunks far from all of its particles (chunk_near); taken
    // here, where few values are live (per segment it would cost registers in the force pass)
    const Box box = CULL ? lane_box(pi, live) : Box{};
    const float lim = h2 * (1.0f + 0x1p-10f);
    const CellXYZ ci = key_xyz(load_or(skeys, s, live, 0u), g);
    uint32_t b[3], e[3];
    slab_ranges(ci, live, g, cstart, n, (int)slab - 1, b, e);
    const uint32_t hr = home_row(ci, g);
    float acc = 0.0f;
    if (trans)  // members take their representative's density
        acc = density_trans(spos, b, e, pi, live && !is_member(__float_as_uint(pi.w), s), h2,
                            trans_lanes(wave, hw), lane);
    uint64_t pending = trans ? 0ull : __ballot(live);
    while (pending) {  // uniform, identical in every wave
        const int leader = __ffsll((unsigned long long)pending) - 1;
        const uint32_t row = (uint32_t)__shfl((int)hr, leader, kWave);
        const bool mine = live && hr == row;
        const uint64_t seg = __ballot(mine);
        pending &= ~seg;
        const int last = 63 - __clzll((long long)seg);
        RowPlan R[3];
        seg_plans(R, ci, g, (int)slab - 1, b, e, leader, last, cut, cstart, cell_grp, epoch,
                  lane);
        // chunks wave, wave + hw, ... of the segment's three rows; the next is fetched before
        // the current one is evaluated; a chunk with no candidate near the item is skipped
        const uint32_t same = CULL ? same_rows(b, e, mine, leader) : 0u;
        uint32_t t = (uint32_t)wave;
        int r;
        uint32_t c0, m;
        seg_chunk(R, t, r, c0, m);
        float4 v = r < 3 ? chunk_load(spos, c0, m, lane) : z4;
        while (r < 3) {  // uniform within the wave
            const uint64_t near = CULL ? near_mask(v, (uint32_t)lane < m, box, lim) : ~0ull;
            const bool go = near != 0ull;
            int nr;
            uint32_t nc0, nm;
            seg_chunk(R, t + (uint32_t)hw, nr, nc0, nm);
            const float4 nv = nr < 3 ? chunk_load(spos, nc0, nm, lane) : z4;
            const uint32_t j = c0 + (uint32_t)lane;
            if (CULL && go && ((same >> r) & 1u)) {  // uniform: the near candidates only
                __builtin_amdgcn_wave_barrier();
                if ((near >> lane) & 1ull)
                    buf[mask_rank(near)] = make_float4(v.x, v.y, v.z, candidate_weight(v.w, j));
                __builtin_amdgcn_wave_barrier();
                const uint32_t k = (uint32_t)__popcll(near);
                if (mine)
                    acc = cut ? density_run_w(buf, 0u, 0u, k, pi, h2, acc)
                              : density_run(buf, 0u, 0u, k, pi, h2, acc);
            } else if (go) {  // uniform
                __builtin_amdgcn_wave_barrier();
                buf[lane] = make_float4(v.x, v.y, v.z, candidate_weight(v.w, j));
                __builtin_amdgcn_wave_barrier();
                if (mine) {
                    const uint32_t jb = max(pick3(b, r), c0), je = min(pick3(e, r), c0 + m);
                    // candidate weights other than 1 only in items that touch a group
                    acc = cut ? density_run_w(buf, c0, jb, je, pi, h2, acc)
                              : density_run(buf, c0, jb, je, pi, h2, acc);
                }
            }
            t += (uint32_t)hw;
            r = nr;
            c0 = nc0;
            m = nm;
            v = nv;
        }
    }
    out = acc;
    return true;
}

// The heavy work partials: part p of heavy entry slot q (the entry's position in its list)
// holds, per lane, kHeavyComps floats at hpart[((q * hw + p) * kHeavyComps + c) * 64 + lane],
// hw = the parts per item (the buffer is sized for kHeavyWavesMax).
__device__ __forceinline__ size_t hpart_at(uint32_t slot, uint32_t hw, int part, int comp,
                                         int lane) {
    return (((size_t)slot * hw + (uint32_t)part) * kHeavyComps + (uint32_t)comp) * 64u +
           (uint32_t)lane;
}

// Heavy entry q of the concatenated lists and its partial-sum slot (slots at or above the
// context's hslot_cap do not exist).
__device__ __forceinline__ uint32_t heavy_entry_slot(const uint32_t* __restrict__ heavy,
                                                     const Control* __restrict__ ctl,
                                                     uint32_t cap, uint32_t q, uint32_t& slot) {
    int k = 0;
    for (; k < kHeavyLists - 1; k++) {
        const uint32_t c = min(ctl->heavy_count[k].v, cap);
        if (q < c) break;
        q -= c;
    }
    slot = heavy_slot((uint32_t)k, q);
    return heavy[(size_t)k * cap + q];
}

// Heavy parts of a pass: workgroups 0 .. hparts - 1 of the pass kernel (hparts = hgrid * P), one
// wave each; the P = hw parts of one heavy entry are workgroups on one XCD (b % 8 is
// the XCD), so they share its L2: b = (q / 8) * 8P + part * 8 + q % 8 for entries q < hgrid, and
// the same workgroup takes q + hgrid, ... after that.  hgrid (a multiple of 8, at most
// kHeavyGrid) follows the item count, so that a small system does not dispatch thousands of
// idle parts (c0's 50,000 particles: 2,346 items).
static_assert(kHeavyGrid % 8 == 0, "heavy part numbering");
// Partial-sum slots of hw parts each in the context's buffer (sized for hslot_cap slots of
// hpart_parts parts): more slots when fewer parts are in use, fewer when more.
static uint32_t slot_cap(const fh_ctx* c, uint32_t hw) {
    const uint64_t room = (uint64_t)c->hslot_cap * c->hpart_parts / hw;
    const uint32_t all = kHeavyLists * c->heavy_cap;
    return room < all ? (uint32_t)room : all;
}
// The largest slot a call of n particles can number (list k, position i: 8i + k), plus one:
// plan workgroup b (kPlanThreads particles, 3 items per 64) appends to list b % kHeavyLists.
static uint32_t slots_needed(uint32_t n) {
    const uint32_t per_list = 3u * (kPlanThreads / 64u) *
                              ceil_div(ceil_div(n, (uint32_t)kPlanThreads), (uint32_t)kHeavyLists);
    return per_list * kHeavyLists;
}
// The pass kernels are compiled for the default part count and for 8.  Unless
// FH_OPT_HEAVY_PARTS fixes it, a call of fewer than kSmallSystemN particles takes 8 when the
// context's uncapped buffer would hold 8 parts for every slot the call can number (its few
// items then make 8 times as many waves): always in a context made for small systems, and in a
// large one, whose buffer for 4 parts of all its items holds 8 parts of a small call's.  The
// choice does not depend on FH_OPT_HEAVY_SLOTS (a cap only moves items to the slot-less walks),
// so capped and uncapped runs split the same way.
static uint32_t heavy_parts(const fh_ctx* c, uint32_t n) {
    if (c->heavy_parts) return c->heavy_parts == 8u ? 8u : (uint32_t)kHeavyWaves;
    const uint64_t room = (uint64_t)kHeavyLists * c->heavy_cap * c->hpart_parts;
    return n < kSmallSystemN && room >= 8ull * slots_needed(n) ? 8u : (uint32_t)kHeavyWaves;
}
// Candidates per particle and slab above which an item is split: FH_OPT_HEAVY_WORK, else 32 for
// small systems (configs[0]: 120 -> 90 us per substep with 8 parts; 24, 28, 36, 40 gave 102, 96,
// 92 and 100 us, every item split 195 us) and 192 otherwise (configs[3]'s trajectory: 412.9 ->
// 406.1 us per substep against 384; 160: 407.8; its fixed state with 96, 128, 224, 256: 418.7,
// 423.5, 410.0, 411.9 us; above 384 a light item's stream no longer fits the two windows kept
// for the force pass: 512 took 729 us).
static uint32_t heavy_work(const fh_ctx* c, uint32_t n) {
    return c->heavy_work ? c->heavy_work : n < kSmallSystemN ? kSmallHeavyWork : kHeavyWork;
}
static uint32_t heavy_grid(uint32_t items) {
    const uint32_t g = (items / 8u + 7u) / 8u * 8u;
    return g < 64u ? 64u : (g > (uint32_t)kHeavyGrid ? (uint32_t)kHeavyGrid : g);
}
__device__ __forceinline__ void heavy_part_of(uint32_t b, uint32_t hw, uint32_t& q0, int& part) {
    q0 = (b / (8u * hw)) * 8u + (b & 7u);
    part = (int)((b >> 3) % hw);
}

// Density pass, one launch: heavy parts first (they are the long work), then one light item per
// wave.  The parts leave their partial sums in hpart; k_prep and k_finalize add them in part
// order.  Held to 8 waves per SIMD (the SGPRs of both paths otherwise limit it to 7; fixed c3
// state 492 -> 489 us per substep).
template <uint32_t HW, bool CULL>
__global__ __attribute__((amdgpu_flat_work_group_size(kWave, kWave), amdgpu_waves_per_eu(8, 8)))
void k_density_pass(
    const float4* __restrict__ spos, const uint32_t* __restrict__ skeys, uint32_t n, GridDesc g,
    const uint32_t* __restrict__ cstart, const uint64_t* __restrict__ cell_grp, float h2,
    float* __restrict__ dpart, uint32_t stride, uint32_t items, const uint8_t* __restrict__ flag,
    const uint32_t* __restrict__ skip_tag, const Control* __restrict__ ctl,
    uint32_t* __restrict__ lstream, uint2* __restrict__ lstream_t,
    const uint32_t* __restrict__ heavy, uint32_t heavy_cap, float* __restrict__ hpart,
    uint32_t hgrid, uint32_t hslot_cap) {
    constexpr uint32_t hw = HW;
    __shared__ float4 s_p[kWin];
    const int lane = threadIdx.x;
    const uint32_t b = blockIdx.x, hparts = hgrid * hw;
    if (b < hparts) {  // uniform
        uint32_t q0;
        int part;
        heavy_part_of(b, hw, q0, part);
        const uint32_t count = heavy_total(ctl, heavy_cap), epoch = ctl->epoch;
        // one walk per step: (entry q, this wave's part) for an item with a partial-sum slot;
        // an item without one (FH_OPT_HEAVY_SLOTS caps them) is walked by its part-0 wave
        // alone, part after part (pn), the parts added in part order through the item's plane
        // (each lane re-reads what it wrote), as k_prep adds a slotted item's (slab_part): the
        // same sums, whichever items got slots
        int pn = 0;
        for (uint32_t q = q0; q < count;) {  // uniform
            uint32_t slot;
            const uint32_t entry = heavy_entry_slot(heavy, ctl, heavy_cap, q, slot);
            const bool slotted = slot < hslot_cap;
            if (!slotted && part != 0) {
                q += hgrid;
                continue;
            }
            const int p = slotted ? part : pn;
            float acc;
            // false in every part or in none (only group members are skipped)
            const bool any = density_heavy_wave<CULL>(entry, p, (int)hw, lane, s_p, spos, skeys,
                                                      n, g, cstart, cell_grp, h2, skip_tag, epoch,
                                                      acc);
            if (any && slotted) {
                hpart[hpart_at(slot, hw, part, 0, lane)] = acc;
            } else if (any) {
                const uint32_t item = entry & ~kEntryFlags;
                const uint32_t s = (item / 3u) * kSub + (uint32_t)lane;
                float* const d = dpart + (size_t)(item % 3u) * stride;
                if (s < n) d[s] = (p == 0 ? 0.0f : d[s]) + acc;
            }
            if (slotted || !any || p + 1 == (int)hw) {
                q += hgrid;
                pn = 0;
            } else {
                pn = p + 1;
            }
        }
        return;
    }
    const uint32_t nl = gridDim.x - hparts;
    density_light(xcd_chunked(b - hparts, nl), lane, s_p, spos, skeys, n, g, cstart, h2,
                  dpart, stride, items, flag, skip_tag, ctl, lstream, lstream_t);
}

// A slab partial of particle j: written to its plane (`plane`, already offset to the slab and
// component) by a light item, or, for a particle of a heavy item (hslot[item] = its list slot),
// the sum of the item's hw part partials of component `comp` in part order.
template <uint32_t HW>
__device__ __forceinline__ float slab_part(const float* __restrict__ plane,
                                           const uint32_t* __restrict__ hslot,
                                           const float* __restrict__ hpart, uint32_t slab,
                                           int comp, uint32_t j) {
    const uint32_t sl = hslot[(j / kSub) * 3u + slab];
    if (sl == kNoSlot) return plane[j];
    float t = 0.0f;
#pragma unroll
    for (int p = 0; p < (int)HW; p++) t += hpart[hpart_at(sl, HW, p, comp, j % kSub)];
    return t;
}

// ---------------------------------------------------------------------------------------------
struct FastForce {
    float h, h2, mc, k, rho0;
    float fp;  // -mass * gcoef / 2: pressure pair term = fp*(p_i+p_j)/rho_j*(h-r)^2/r * (x_i-x_j)
    float fv;  // mu * mass * lcoef: viscosity pair term = fv/rho_j*(h-r) * (v_j-v_i)
    float fr;  // fv / fp (0 when fp = 0, i.e. mass = 0, where fv = 0 as well)
};

template <uint32_t HW>
__device__ __forceinline__ float rho_of(const float* __restrict__ dpart, uint32_t stride,
                                        uint32_t j, float mc, const uint32_t* __restrict__ hslot,
                                        const float* __restrict__ hpart) {
    return mc * ((slab_part<HW>(dpart, hslot, hpart, 0u, 0, j) +
                  slab_part<HW>(dpart + stride, hslot, hpart, 1u, 0, j)) +
                 slab_part<HW>(dpart + 2u * stride, hslot, hpart, 2u, 0, j));
}

// Force records, made once per substep after the density pass (k_prep), one pair per sorted
// particle j: rec[j] = (x, y, z, A_j p_j) and rec[stride + j] = (fv u / rho_j, A_j) with
// A_j = fp w / rho_j, where w is the candidate weight (1; M for the representative of a
// co-located group; 0 for the other members, which the representative stands for) and u = w v_j
// (the group's summed velocity for a representative).  The pressure factor of a pair is then
// one fused multiply-add, p_i A_j + A_j p_j = fp (p_i + p_j) w / rho_j, and the constants fp and
// fv are folded in once per particle instead of once per pair.  1/rho_j is taken as 0 when
// rho_j < 1e-6, which removes the pair like the skip of sph_fused.rs:607.  A non-finite position is recorded far away (1e30), so no pair
// with it passes the distance test and the branch-free pair loop never multiplies by NaN.
// srho[j] = rho_j; members take their representative's density (they sit at its position).
// The force kernels then only copy records into LDS.
template <uint32_t HW>
__global__ __launch_bounds__(256) void k_prep(const float4* __restrict__ spos,
                                              const float4* __restrict__ svel,
                                              const float4* __restrict__ vrep,
                                              const float* __restrict__ dpart, uint32_t n,
                                              uint32_t stride, float mc, float k, float rho0,
                                              float fp, float fv, float* __restrict__ srho,
                                              float4* __restrict__ rec,
                                              const uint32_t* __restrict__ hslot,
                                              const float* __restrict__ hpart) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const float4 p = spos[s];
    const uint32_t wb = __float_as_uint(p.w);
    uint32_t r = s;
    float wt = 1.0f;
    float4 u = svel[s];
    if (wb & kRepFlag) {
        wt = (float)(wb & ~kRepFlag);
        u = vrep[s];
    } else if (wb != s) {  // member of a co-located group: wb is its representative
        r = wb < n ? wb : s;
        wt = 0.0f;
        u = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    const float rho = rho_of<HW>(dpart, stride, r, mc, hslot, hpart);
    const float inv = rho < 1e-6f ? 0.0f : 1.0f / rho;
    srho[s] = rho;
    const bool fin = isfinite(p.x) && isfinite(p.y) && isfinite(p.z);
    const float A = fp * (wt * inv), vi = fv * inv;
    rec[s] = fin ? make_float4(p.x, p.y, p.z, A * (k * (rho - rho0)))
                 : make_float4(1e30f, 1e30f, 1e30f, 0.0f);
    rec[stride + s] = make_float4(u.x * vi, u.y * vi, u.z * vi, A);
}

// Pressure + viscosity pair terms of one lane over [jb, je) of staged records (k_prep):
// per candidate  (p_i A_j + A_j p_j) (h - r)^2 / r (x_i - x_j) + (h - r) (fv u_j / rho_j), and
// wa += (h - r) A_j; the weight of -v_i in the viscosity sum is fr * wa (applied once by the
// caller).  Branch-free: the pair test selects the scale factors, so the loads of the next
// candidates issue ahead of the arithmetic; staged positions are finite (k_prep) and the
// pressure factor is selected after its product, so a non-pair (r = 0 included) adds exact zeros.
__device__ __forceinline__ void force_pair(const float4& q, const float4& w, const float4& pi,
                                           float p_i, const FastForce& K, float& ax, float& ay,
                                           float& az, float& wa) {
    const float dx = pi.x - q.x, dy = pi.y - q.y, dz = pi.z - q.z;
    // r^2 + 1e-30: identical for every pair that passes the test (r^2 > 1e-12), and never 0, so
    // 1/r stays finite and a rejected pair's zeroed (h - r) zeroes its pressure factor as well
    // (one select instead of two)
    const float r2 = fmaf(dz, dz, fmaf(dy, dy, fmaf(dx, dx, 1e-30f)));
    const bool ok = r2 < K.h2 && r2 > 1e-12f;
    // The empty asm pins 1/r as computed for every candidate: otherwise the compiler moves the
    // reciprocal square root and the products behind a divergent branch on the pair test, whose
    // exec-mask bookkeeping costs more than the select (10% of the light force work on c3).
    float rinv = __builtin_amdgcn_rsqf(r2);
    asm volatile("" : "+v"(rinv));
    const float vs = ok ? fmaf(-r2, rinv, K.h) : 0.0f;
    const float fs = (fmaf(p_i, w.w, q.w) * vs) * (vs * rinv);
    wa = fmaf(vs, w.w, wa);
    ax = fmaf(vs, w.x, fmaf(fs, dx, ax));
    ay = fmaf(vs, w.y, fmaf(fs, dy, ay));
    az = fmaf(vs, w.z, fmaf(fs, dz, az));
}

// U candidates per iteration (their loads issued together).
template <int U>
__device__ __forceinline__ void force_run(const float4* __restrict__ sp,
                                          const float4* __restrict__ sv, uint32_t c0,
                                          uint32_t jb, uint32_t je, float4 pi, float p_i,
                                          const FastForce& K, float& ax, float& ay, float& az,
                                          float& wv) {
    // pointer-stepped: the loop keeps one address and one compare per U candidates; empty when
    // je <= jb (je may lie before the chunk, where je - c0 would wrap around)
    const uint32_t m = je > jb ? je - jb : 0u;
    const float4* p = sp + (jb - c0);
    const float4* v = sv + (jb - c0);
    const float4* const pe = p + m;
    if (U > 1) {
        // p < pu: U more candidates (bounds from the count, as in density_run)
        const float4* const pu = p + (m > (uint32_t)(U - 1) ? m - (uint32_t)(U - 1) : 0u);
        if (p < pu) {
            do {
                float4 q[U], w[U];
#pragma unroll
                for (int u = 0; u < U; u++) {
                    q[u] = p[u];
                    w[u] = v[u];
                }
#pragma unroll
                for (int u = 0; u < U; u++) force_pair(q[u], w[u], pi, p_i, K, ax, ay, az, wv);
                p += U;
                v += U;
            } while (p < pu);
        }
    }
    for (; p < pe; p++, v++) force_pair(*p, *v, pi, p_i, K, ax, ay, az, wv);
}

// Transposed force walk of the item's particles taken by this wave: in the lane of each such
// particle, its acceleration partial (a_x, a_y, a_z) and viscosity weight sum wa (force_pair).
__device__ __forceinline__ void force_trans(const float4* __restrict__ rec,
                                            const float4* __restrict__ spos, uint32_t stride,
                                            const uint32_t b[3], const uint32_t e[3],
                                            const float4& pi, float p_i, bool mine,
                                            const FastForce& K, uint64_t lanes, int lane,
                                            float& oax, float& oay, float& oaz, float& owa) {
    uint64_t todo = __ballot(mine) & lanes;
    while (todo) {  // uniform
        const int l = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1ull;
        const float4 pl = make_float4(__shfl(pi.x, l, kWave), __shfl(pi.y, l, kWave),
                                      __shfl(pi.z, l, kWave), 0.0f);
        const float pp = __shfl(p_i, l, kWave);
        float ax = 0.0f, ay = 0.0f, az = 0.0f, wa = 0.0f;
#pragma unroll
        for (int r = 0; r < 3; r++) {
            const uint32_t bb = (uint32_t)__shfl((int)b[r], l, kWave);
            const uint32_t ee = (uint32_t)__shfl((int)e[r], l, kWave);
            for (uint32_t j0 = bb; j0 < ee;) {  // uniform
                const uint32_t j = j0 + (uint32_t)lane;
                const bool ok = j < ee;
                const uint32_t jj = ok ? j : j0;
                float4 q = rec[jj], w = rec[stride + jj];
                const uint32_t wb = __float_as_uint(spos[jj].w);
                if (!ok) {  // adds zeros
                    q.w = 0.0f;
                    w = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                force_pair(q, w, pl, pp, K, ax, ay, az, wa);
                j0 = trans_next(j0, j, ok, wb);
            }
        }
        ax = wave_sum(ax);
        ay = wave_sum(ay);
        az = wave_sum(az);
        wa = wave_sum(wa);
        if (lane == l) {
            oax = ax;
            oay = ay;
            oaz = az;
            owa = wa;
        }
    }
}

// Acceleration partials: fpart[slab][c][s] = sum over the slab's neighbours j of the pressure
// and viscosity pair terms (sph_fused.rs:604-623), not yet divided by rho_i.  Same windowed
// stream as density_light; the window is staged by copying force records (k_prep).
__device__ __forceinline__ void force_light(uint32_t item, int lane, float4* bp, float4* bv,
                                            const float4* __restrict__ spos,
                                            const float4* __restrict__ svel,
                                            const float* __restrict__ srho,
                                            const float4* __restrict__ rec,
                                            const uint32_t* __restrict__ skeys, uint32_t n,
                                            GridDesc g, const uint32_t* __restrict__ cstart,
                                            const FastForce& K, float* __restrict__ fpart,
                                            float* __restrict__ wpart, uint32_t stride,
                                            uint32_t items, const uint8_t* __restrict__ flag,
                                            const uint32_t* __restrict__ skip_tag,
                                            const Control* __restrict__ ctl,
                                            const uint32_t* __restrict__ lstream,
                                            const uint2* __restrict__ lstream_t) {
    if (item >= items || flag[item] != kItemLight) return;  // whole wave
    const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
    if (skip_tag[sub] == ctl->epoch) return;  // only group members (finished from the group)
    const uint32_t s = sub * kSub + (uint32_t)lane;
    const bool in = s < n;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 pi = load_or(spos, s, in, z4);
    const float4 vi = load_or(svel, s, in, z4);
    const float rho_i = load_or(srho, s, in, 0.0f);
    const bool live = in && !(rho_i < 1e-6f);  // sph_fused.rs:550
    const float p_i = K.k * (rho_i - K.rho0);
    // the candidate stream the density pass left (short streams), else rebuilt
    LightStream L;
    const uint2 tb = lstream_t[item];
    L.T = tb.x;
    const bool kept = tb.y != kNoBase;  // uniform
    const uint32_t* lc = lstream + (size_t)item * kLightCacheWords;
    if (kept) {
        get_intervals(lc, lane, L);
    } else {
        const CellXYZ ci = key_xyz(load_or(skeys, s, in, 0u), g);
        uint32_t b[3], e[3];
        slab_ranges(ci, in, g, cstart, n, (int)slab - 1, b, e);
        light_stream(L, b, e, home_row(ci, g), in, lane);
    }
    float ax = 0.0f, ay = 0.0f, az = 0.0f, wv = 0.0f;
    for (uint32_t w0 = 0; w0 < L.T; w0 += kWin) {  // wave-uniform
        uint32_t j[kWinLoads];
        if (kept) {
            get_offsets(lc + kLightHead, w0, lane, j, tb.y);
        } else {
            window_indices(L, w0, lane, j);
        }
        float4 q[kWinLoads], w[kWinLoads];
#pragma unroll
        for (int k = 0; k < kWinLoads; k++) {
            q[k] = rec[j[k]];
            w[k] = rec[stride + j[k]];
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int k = 0; k < kWinLoads; k++) {
            bp[k * kWave + lane] = q[k];
            bv[k * kWave + lane] = w[k];
        }
        __builtin_amdgcn_wave_barrier();
        if (live) {
            uint32_t jb[3], je[3];
            window_rows(L, w0, jb, je);
#pragma unroll
            for (int r = 0; r < 3; r++)
                if (jb[r] < je[r]) force_run<4>(bp, bv, w0, jb[r], je[r], pi, p_i, K, ax, ay, az, wv);
        }
    }
    if (in) {
        wv *= K.fr;
        float* o = fpart + (size_t)slab * 3u * stride;
        o[s] = fmaf(-wv, vi.x, ax);
        o[stride + s] = fmaf(-wv, vi.y, ay);
        o[2u * (size_t)stride + s] = fmaf(-wv, vi.z, az);
        // a group representative's viscosity weight for this slab (k_finalize finishes its
        // members with it); every slab of a representative is written by one of the two kernels
        if (__float_as_uint(pi.w) & kRepFlag) wpart[(size_t)slab * stride + s] = wv;
    }
}

// One virtual wave (`wave` of hw) of heavy entry `entry` in the force pass: its partial
// acceleration (with the -wv v_i viscosity part, which adds linearly) and viscosity weight.
// False when the item is skipped (only group members).
template <bool CULL>
__device__ __forceinline__ bool force_heavy_wave(
    uint32_t entry, int wave, int hw, int lane, float4* bp, float4* bv, const float4* __restrict__ spos,
    const float4* __restrict__ svel, const float* __restrict__ srho,
    const float4* __restrict__ rec, const uint32_t* __restrict__ skeys, uint32_t n, GridDesc g,
    const uint32_t* __restrict__ cstart, const uint64_t* __restrict__ cell_grp,
    const FastForce& K, uint32_t stride, const uint32_t* __restrict__ skip_tag, uint32_t epoch,
    float out[4]) {
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const bool cut = (entry & kCutFlag) != 0u;
    const bool trans = (entry & kTransFlag) != 0u;
    const uint32_t item = entry & ~kEntryFlags;
    const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
    if (skip_tag[sub] == epoch) return false;  // uniform: only group members
    const uint32_t s = sub * kSub + (uint32_t)lane;
    const bool in = s < n;
    const float4 pi = load_or(spos, s, in, z4);
    const float rho_i = load_or(srho, s, in, 0.0f);
    const bool live = in && !(rho_i < 1e-6f);
    const float p_i = K.k * (rho_i - K.rho0);
    const Box box = CULL ? lane_box(pi, live) : Box{};  // as in density_heavy_wave
    const float lim = K.h2 * (1.0f + 0x1p-10f);
    const CellXYZ ci = key_xyz(load_or(skeys, s, in, 0u), g);
    uint32_t b[3], e[3];
    slab_ranges(ci, live, g, cstart, n, (int)slab - 1, b, e);
    const uint32_t hr = home_row(ci, g);
    float ax = 0.0f, ay = 0.0f, az = 0.0f, wv = 0.0f;
    if (trans)  // members are finished from their representative
        force_trans(rec, spos, stride, b, e, pi, p_i,
                    live && !is_member(__float_as_uint(pi.w), s), K, trans_lanes(wave, hw), lane,
                    ax, ay, az, wv);
    uint64_t pending = trans ? 0ull : __ballot(live);
    while (pending) {  // uniform, identical in every wave
        const int leader = __ffsll((unsigned long long)pending) - 1;
        const uint32_t row = (uint32_t)__shfl((int)hr, leader, kWave);
        const bool mine = live && hr == row;
        const uint64_t seg = __ballot(mine);
        pending &= ~seg;
        const int last = 63 - __clzll((long long)seg);
        RowPlan R[3];
        seg_plans(R, ci, g, (int)slab - 1, b, e, leader, last, cut, cstart, cell_grp, epoch,
                  lane);
        const uint32_t same = CULL ? same_rows(b, e, mine, leader) : 0u;  // as in density
        uint32_t t = (uint32_t)wave;
        int r;
        uint32_t c0, m;
        seg_chunk(R, t, r, c0, m);
        // records of chunk t (lanes past the chunk load a valid index; their slots are never
        // read), the next chunk's fetched before the current one is evaluated
        float4 q = load_or(rec, c0 + min((uint32_t)lane, m - 1u), r < 3, z4);
        float4 w = load_or(rec + stride, c0 + min((uint32_t)lane, m - 1u), r < 3, z4);
        while (r < 3) {  // uniform within the wave
            // a chunk with no record near the item is skipped (chunk_near); decided before
            // the next chunk's loads are issued, so its temporaries are not live beside them
            const uint64_t near = CULL ? near_mask(q, (uint32_t)lane < m, box, lim) : ~0ull;
            const bool go = near != 0ull;
            int nr;
            uint32_t nc0, nm;
            seg_chunk(R, t + (uint32_t)hw, nr, nc0, nm);
            const float4 nq = load_or(rec, nc0 + min((uint32_t)lane, nm - 1u), nr < 3, z4);
            const float4 nw = load_or(rec + stride, nc0 + min((uint32_t)lane, nm - 1u), nr < 3, z4);
            if (CULL && go && ((same >> r) & 1u)) {  // uniform: the near records only
                __builtin_amdgcn_wave_barrier();
                if ((near >> lane) & 1ull) {
                    const uint32_t x = mask_rank(near);
                    bp[x] = q;
                    bv[x] = w;
                }
                __builtin_amdgcn_wave_barrier();
                if (mine)
                    force_run<FH_HU>(bp, bv, 0u, 0u, (uint32_t)__popcll(near), pi, p_i, K, ax, ay,
                                     az, wv);
            } else if (go) {  // uniform
                __builtin_amdgcn_wave_barrier();
                bp[lane] = q;
                bv[lane] = w;
                __builtin_amdgcn_wave_barrier();
                if (mine)
                    force_run<CULL ? FH_HU : 2 * FH_HU>(bp, bv, c0, max(pick3(b, r), c0),
                                                        min(pick3(e, r), c0 + m), pi, p_i, K, ax,
                                                        ay, az, wv);
            }
            t += (uint32_t)hw;
            r = nr;
            c0 = nc0;
            m = nm;
            q = nq;
            w = nw;
        }
    }
    // the -wv v_i part of the viscosity sum (wave partials add linearly)
    wv *= K.fr;
    const float4 vi = load_or(svel, s, in, z4);
    out[0] = fmaf(-wv, vi.x, ax);
    out[1] = fmaf(-wv, vi.y, ay);
    out[2] = fmaf(-wv, vi.z, az);
    out[3] = wv;
    return true;
}

// Force pass, one launch: heavy parts first, then one light item per wave (as k_density_pass).
// Held to 6 waves per SIMD (80 registers): the light rows take 4 candidates per step (4 loads in
// flight; 2 per step at 7 waves: c3's fixed state 167.9 instead of 163.6 us), and the chunk tests
// (CULL) fit without spilling (at 7 waves they spill 2 registers: 3 % slower on configs[4]).
template <uint32_t HW, bool CULL>
__global__ __launch_bounds__(kWave) __attribute__((amdgpu_waves_per_eu(6, 8))) void k_force_pass(
    const float4* __restrict__ spos, const float4* __restrict__ svel,
    const float* __restrict__ srho, const float4* __restrict__ rec,
    const uint32_t* __restrict__ skeys, uint32_t n, GridDesc g,
    const uint32_t* __restrict__ cstart, const uint64_t* __restrict__ cell_grp, FastForce K,
    float* __restrict__ fpart, float* __restrict__ wpart, uint32_t stride, uint32_t items,
    const uint8_t* __restrict__ flag, const uint32_t* __restrict__ skip_tag,
    const Control* __restrict__ ctl, const uint32_t* __restrict__ lstream,
    const uint2* __restrict__ lstream_t, const uint32_t* __restrict__ heavy,
    uint32_t heavy_cap, float* __restrict__ hpart, uint32_t hgrid, uint32_t hslot_cap) {
    constexpr uint32_t hw = HW;
    __shared__ float4 s_p[kWin];  // x, y, z, p_j
    __shared__ float4 s_v[kWin];  // u/rho_j, w/rho_j
    const int lane = threadIdx.x;
    const uint32_t b = blockIdx.x, hparts = hgrid * hw;
    if (b < hparts) {  // uniform
        uint32_t q0;
        int part;
        heavy_part_of(b, hw, q0, part);
        const uint32_t count = heavy_total(ctl, heavy_cap), epoch = ctl->epoch;
        // one walk per step: (entry q, this wave's part) for an item with a partial-sum slot;
        // an item without one (FH_OPT_HEAVY_SLOTS caps them) is walked by its part-0 wave
        // alone, part after part (pn), the parts added in part order through the item's planes
        // (each lane re-reads what it wrote), as k_finalize adds a slotted item's (slab_part):
        // the same sums, whichever items got slots
        int pn = 0;
        for (uint32_t q = q0; q < count;) {  // uniform
            uint32_t slot;
            const uint32_t entry = heavy_entry_slot(heavy, ctl, heavy_cap, q, slot);
            const bool slotted = slot < hslot_cap;
            if (!slotted && part != 0) {
                q += hgrid;
                continue;
            }
            const int p = slotted ? part : pn;
            float o[4];
            // false in every part or in none (only group members are skipped)
            const bool any = force_heavy_wave<CULL>(entry, p, (int)hw, lane, s_p, s_v, spos, svel,
                                                    srho, rec, skeys, n, g, cstart, cell_grp, K,
                                                    stride, skip_tag, epoch, o);
            if (any && slotted) {
#pragma unroll
                for (int c = 0; c < 4; c++) hpart[hpart_at(slot, hw, part, c, lane)] = o[c];
            } else if (any) {
                const uint32_t item = entry & ~kEntryFlags;
                const uint32_t s = (item / 3u) * kSub + (uint32_t)lane;
                float* const f = fpart + (size_t)(item % 3u) * 3u * stride;
                float* const wp = wpart + (size_t)(item % 3u) * stride;
                if (s < n) {
                    const bool first = p == 0;
                    f[s] = (first ? 0.0f : f[s]) + o[0];
                    f[stride + s] = (first ? 0.0f : f[stride + s]) + o[1];
                    f[2u * (size_t)stride + s] = (first ? 0.0f : f[2u * (size_t)stride + s]) + o[2];
                    // read only for a group representative (k_finalize finishes its members)
                    wp[s] = (first ? 0.0f : wp[s]) + o[3];
                }
            }
            if (slotted || !any || p + 1 == (int)hw) {
                q += hgrid;
                pn = 0;
            } else {
                pn = p + 1;
            }
        }
        return;
    }
    const uint32_t nl = gridDim.x - hparts;
    force_light(xcd_chunked(b - hparts, nl), lane, s_p, s_v, spos, svel, srho, rec, skeys, n,
                g, cstart, K, fpart, wpart, stride, items, flag, skip_tag, ctl, lstream,
                lstream_t);
}

// ---------------------------------------------------------------------------------------------
struct Finish {
    float mc, dt;
    uint32_t flags;  // FH_EPI_* ; bit 31: density only (no force partials, no state update)
    float gx, gy, gz;
    float mn[3], mx[3], e;
};
constexpr uint32_t kDensityOnly = 1u << 31;

// Sum the slab partials, apply v += a dt and the fused epilogue (gravity.rs:33,
// integrate.rs:23-29, box_collider.rs:37-46), in sorted order: the new state of particle s goes
// to sout[2 s] = (x, y, z, rho) and sout[2 s + 1] = (vx, vy, vz, bits of the particle id) (32
// contiguous bytes) and,
// when accelerations are asked for, to sout[2 stride + s] = (ax, ay, az, 0).  k_scatter then
// moves it to particle order.
template <uint32_t HW>
__global__ __launch_bounds__(256) void k_finalize(const float4* __restrict__ spos,
                                                  const float4* __restrict__ svel,
                                                  const float* __restrict__ dpart,
                                                  const float* __restrict__ fpart,
                                                  const float* __restrict__ wpart, uint32_t n,
                                                  uint32_t stride, Finish F, bool want_accel,
                                                  float4* __restrict__ sout, GridDesc g,
                                                  uint32_t* __restrict__ keys_out,
                                                  const uint32_t* __restrict__ hslot,
                                                  const float* __restrict__ hpart,
                                                  const float* __restrict__ srho,
                                                  uint32_t* __restrict__ rank_out) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const float4 p = spos[s];
    // Co-located particle: its density, and its acceleration up to the viscosity term, are
    // those of its representative r; sum_j w_j (v_j - v_s) = [sum_j w_j (v_j - v_r)] + W (v_r - v_s)
    // with W = sum_j w_j, which the force pass kept for r.
    const uint32_t wb = __float_as_uint(p.w);
    uint32_t r = (wb & kRepFlag) ? s : wb;
    if (r >= n) r = s;
    // after a force pass k_prep has left rho (of r) in srho, and the force pass has reused the
    // heavy parts' partial buffer, so the density partials are summed only when density is all
    const float rho = (F.flags & kDensityOnly) ? rho_of<HW>(dpart, stride, r, F.mc, hslot, hpart)
                                               : srho[s];
    if (F.flags & kDensityOnly) {
        sout[2u * s] = make_float4(p.x, p.y, p.z, rho);
        return;
    }
    const float4 v = svel[s];
    float ax = 0.0f, ay = 0.0f, az = 0.0f;
    float nvx = v.x, nvy = v.y, nvz = v.z;
    if (!(rho < 1e-6f)) {
        const float inv = 1.0f / rho;
        const size_t S = stride;
        float fx = (slab_part<HW>(fpart, hslot, hpart, 0u, 0, r) +
                    slab_part<HW>(fpart + 3 * S, hslot, hpart, 1u, 0, r)) +
                   slab_part<HW>(fpart + 6 * S, hslot, hpart, 2u, 0, r);
        float fy = (slab_part<HW>(fpart + S, hslot, hpart, 0u, 1, r) +
                    slab_part<HW>(fpart + 4 * S, hslot, hpart, 1u, 1, r)) +
                   slab_part<HW>(fpart + 7 * S, hslot, hpart, 2u, 1, r);
        float fz = (slab_part<HW>(fpart + 2 * S, hslot, hpart, 0u, 2, r) +
                    slab_part<HW>(fpart + 5 * S, hslot, hpart, 1u, 2, r)) +
                   slab_part<HW>(fpart + 8 * S, hslot, hpart, 2u, 2, r);
        if (r != s) {
            const float W = (slab_part<HW>(wpart, hslot, hpart, 0u, 3, r) +
                             slab_part<HW>(wpart + S, hslot, hpart, 1u, 3, r)) +
                            slab_part<HW>(wpart + 2 * S, hslot, hpart, 2u, 3, r);
            const float4 vr = svel[r];
            fx = fmaf(W, vr.x - v.x, fx);
            fy = fmaf(W, vr.y - v.y, fy);
            fz = fmaf(W, vr.z - v.z, fz);
        }
        ax = fx * inv;
        ay = fy * inv;
        az = fz * inv;
        nvx = v.x + ax * F.dt;
        nvy = v.y + ay * F.dt;
        nvz = v.z + az * F.dt;
    }
    float npx = p.x, npy = p.y, npz = p.z;
    if (F.flags & FH_EPI_GRAVITY) {
        nvx += F.gx * F.dt;
        nvy += F.gy * F.dt;
        nvz += F.gz * F.dt;
    }
    if (F.flags & FH_EPI_INTEGRATE) {
        if (!isfinite(nvx)) nvx = 0.0f;
        if (!isfinite(nvy)) nvy = 0.0f;
        if (!isfinite(nvz)) nvz = 0.0f;
        npx += nvx * F.dt;
        npy += nvy * F.dt;
        npz += nvz * F.dt;
    }
    if (F.flags & FH_EPI_BOX) {
        if (npx < F.mn[0]) { npx = F.mn[0]; nvx = fabsf(nvx) * F.e; }
        if (npx > F.mx[0]) { npx = F.mx[0]; nvx = -fabsf(nvx) * F.e; }
        if (npy < F.mn[1]) { npy = F.mn[1]; nvy = fabsf(nvy) * F.e; }
        if (npy > F.mx[1]) { npy = F.mx[1]; nvy = -fabsf(nvy) * F.e; }
        if (npz < F.mn[2]) { npz = F.mn[2]; nvz = fabsf(nvz) * F.e; }
        if (npz > F.mx[2]) { npz = F.mx[2]; nvz = -fabsf(nvz) * F.e; }
    }
    sout[2u * s] = make_float4(npx, npy, npz, rho);
    sout[2u * s + 1u] = make_float4(nvx, nvy, nvz, v.w);  // .w: the particle id
    if (keys_out) keys_out[s] = sort_key_of(npx, npy, npz, g);  // the next resident substep's keys
    // the last of several resident substeps: the particle -> slot map for k_scatter (what
    // k_rank_of would read back from the new state)
    if (rank_out && __float_as_uint(v.w) < n) rank_out[__float_as_uint(v.w)] = s;
    if (want_accel) sout[2 * (size_t)stride + s] = make_float4(ax, ay, az, 0.0f);
}

// Particle order: particle i reads its new state at its sorted position rank[i] (one 32-byte
// read) and writes the caller's arrays coalesced.  Positions are written only when the
// epilogue moves them.
__global__ __launch_bounds__(256) void k_scatter(const float4* __restrict__ sout,
                                                 const uint32_t* __restrict__ rank, uint32_t n,
                                                 uint32_t stride, uint32_t flags,
                                                 float* __restrict__ px, float* __restrict__ py,
                                                 float* __restrict__ pz, float* __restrict__ vx,
                                                 float* __restrict__ vy, float* __restrict__ vz,
                                                 float* __restrict__ density,
                                                 float* __restrict__ accel) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t r = rank[i];
    if (r >= n) return;  // never taken when the sort is consistent
    const float4 o0 = sout[2u * r];
    if (density) density[i] = o0.w;
    if (flags & kDensityOnly) return;
    const float4 o1 = sout[2u * r + 1u];
    vx[i] = o1.x;
    vy[i] = o1.y;
    vz[i] = o1.z;
    if (flags & (FH_EPI_INTEGRATE | FH_EPI_BOX)) {
        px[i] = o0.x;
        py[i] = o0.y;
        pz[i] = o0.z;
    }
    if (accel) {
        const float4 o2 = sout[2 * (size_t)stride + r];
        accel[i] = o2.x;
        accel[(size_t)n + i] = o2.y;
        accel[2 * (size_t)n + i] = o2.z;
    }
}

// ---------------------------------------------------------------------------------------------
// Light kernels: one (64-particle sub-tile, slab) item per wave, 4 waves per workgroup.
static uint32_t wave_grid(uint32_t n, uint32_t* items) {
    *items = ceil_div(n, (uint32_t)kSub) * 3u;
    return ceil_div(*items, (uint32_t)(kTileP / kWave));
}

static float poly6_mc(float h, float mass) {
    // sph_density.rs:413-416 and the leading `mass * poly6_coeff` product of :453
    float h2 = h * h;
    float h9 = h2 * h2 * h2 * h2 * h;
    float poly6 = 315.0f / (64.0f * 3.14159265f * h9);
    return mass * poly6;
}



hipError_t launch_group_plan(fh_ctx* c, const SphArgs& a, bool with_vel) {
    if (a.n == 0) return hipSuccess;
    // scratch of the group part: the sort's key buffer, free after the sort (disjoint ranges per cell)
    tbeg(c, KID_PLAN);
    k_group_plan<<<kGroupBlocks + ceil_div(a.n, (uint32_t)kPlanThreads), kPlanThreads, 0,
                   c->stream>>>(c->big, ceil_div(c->max_n, 64u) + 1u, a.n, c->skeys, c->cell_start,
                                c->spos, with_vel ? c->svel : nullptr, c->sidx, c->rank, c->ka,
                                c->cell_grp, c->vrep, c->skip_tag, a.g, c->run_tag,
                                c->heavy_flag, c->heavy, c->heavy_cap,
                                heavy_work(c, a.n), c->direct_mode,
                                c->ctl, c->lstream, c->lstream_t, c->hslot,
                                slot_cap(c, heavy_parts(c, a.n)));
    tend(c, KID_PLAN);
    return hipGetLastError();
}

hipError_t launch_density_fast(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start) {
    if (a.n == 0) return hipSuccess;
    uint32_t items;
    const uint32_t grid = wave_grid(a.n, &items);
    tbeg(c, KID_DENSITY);
    const uint32_t hgrid = heavy_grid(items);
    const uint32_t hw = heavy_parts(c, a.n);
    // the heavy walks skip far chunks only where the cells are ordered by sub-cell (g.sb > 0)
    const bool cull = a.g.sb != 0u;
    const auto kernel = hw == 8u ? (cull ? k_density_pass<8, true> : k_density_pass<8, false>)
                                 : (cull ? k_density_pass<kHeavyWaves, true>
                                         : k_density_pass<kHeavyWaves, false>);
    kernel<<<hgrid * hw + grid, kWave, 0, c->stream>>>(
        c->spos, c->skeys, a.n, a.g, cell_start, c->cell_grp, a.h * a.h, c->dpart, c->max_n,
        items, c->heavy_flag, c->skip_tag, c->ctl, c->lstream, c->lstream_t, c->heavy,
        c->heavy_cap, c->hpart, hgrid, slot_cap(c, hw));
    hipError_t e = hipGetLastError();
    tend(c, KID_DENSITY);
    return e;
}


static FastForce fast_force(const SphArgs& a) {
    FastForce K;
    K.h = a.h;
    K.h2 = a.h * a.h;
    K.mc = poly6_mc(a.h, a.mass);
    K.k = a.k;
    K.rho0 = a.rho0;
    const float h6 = K.h2 * K.h2 * K.h2;
    const float gcoef = -45.0f / (3.14159265f * h6);  // sph_fused.rs:554
    const float lcoef = 45.0f / (3.14159265f * h6);   // sph_fused.rs:555
    K.fp = -a.mass * gcoef * 0.5f;
    K.fv = a.mu * a.mass * lcoef;
    K.fr = K.fp != 0.0f ? K.fv / K.fp : 0.0f;
    return K;
}

hipError_t launch_prep(fh_ctx* c, const SphArgs& a) {
    if (a.n == 0) return hipSuccess;
    const FastForce K = fast_force(a);
    tbeg(c, KID_PREP);
    const auto kernel = heavy_parts(c, a.n) == 8u ? k_prep<8> : k_prep<kHeavyWaves>;
    kernel<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->spos, c->svel, c->vrep, c->dpart, a.n,
                                                       c->max_n, K.mc, a.k, a.rho0, K.fp, K.fv,
                                                       c->srho, c->sout, c->hslot, c->hpart);
    tend(c, KID_PREP);
    return hipGetLastError();
}

hipError_t launch_force_fast(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start) {
    if (a.n == 0) return hipSuccess;
    const FastForce K = fast_force(a);
    uint32_t items;
    const uint32_t grid = wave_grid(a.n, &items);
    tbeg(c, KID_FORCE);
    const uint32_t hgrid = heavy_grid(items);
    const uint32_t hw = heavy_parts(c, a.n);
    const bool cull = a.g.sb != 0u;  // as in launch_density_fast
    const auto kernel = hw == 8u ? (cull ? k_force_pass<8, true> : k_force_pass<8, false>)
                                 : (cull ? k_force_pass<kHeavyWaves, true>
                                         : k_force_pass<kHeavyWaves, false>);
    kernel<<<hgrid * hw + grid, kWave, 0, c->stream>>>(
        c->spos, c->svel, c->srho, c->sout, c->skeys, a.n, a.g, cell_start, c->cell_grp, K,
        c->fpart, c->wpart, c->max_n, items, c->heavy_flag, c->skip_tag, c->ctl, c->lstream,
        c->lstream_t, c->heavy, c->heavy_cap, c->hpart, hgrid, slot_cap(c, hw));
    hipError_t e = hipGetLastError();
    tend(c, KID_FORCE);
    return e;
}

// rank[id] = s for the particle id carried in the new state of slot s (sout[2 s + 1].w): the
// particle -> slot map after resident substeps.
__global__ __launch_bounds__(256) void k_rank_of(const float4* __restrict__ sout, uint32_t n,
                                                 uint32_t* __restrict__ rank) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const uint32_t i = __float_as_uint(sout[2u * s + 1u].w);
    if (i < n) rank[i] = s;
}

hipError_t launch_finalize(fh_ctx* c, const SphArgs& a, const fh_epilogue* epi, bool density_only,
                           float* px, float* py, float* pz, float* vx, float* vy, float* vz,
                           float* density, float* accel, bool to_particles, bool rebuild_rank,
                           uint32_t* next_keys) {
    if (a.n == 0) return hipSuccess;
    Finish F;
    F.mc = poly6_mc(a.h, a.mass);
    F.dt = a.dt;
    F.flags = (epi ? epi->flags : 0u) | (density_only ? kDensityOnly : 0u);
    F.gx = epi ? epi->gravity[0] : 0.0f;
    F.gy = epi ? epi->gravity[1] : 0.0f;
    F.gz = epi ? epi->gravity[2] : 0.0f;
    for (int q = 0; q < 3; q++) {
        F.mn[q] = epi ? epi->box_min[q] : 0.0f;
        F.mx[q] = epi ? epi->box_max[q] : 0.0f;
    }
    F.e = epi ? epi->restitution : 0.0f;
    tbeg(c, KID_FINAL);
    // after resident substeps k_finalize itself writes the particle -> slot map (with forces: a
    // density-only call returns before it has the particle id)
    const bool rank_here = to_particles && rebuild_rank && !density_only;
    const auto fin = heavy_parts(c, a.n) == 8u ? k_finalize<8> : k_finalize<kHeavyWaves>;
    fin<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->spos, c->svel, c->dpart, c->fpart,
                                                           c->wpart, a.n, c->max_n, F,
                                                           accel != nullptr, c->sout, a.g,
                                                           density_only ? nullptr : next_keys,
                                                           c->hslot, c->hpart, c->srho,
                                                           rank_here ? c->rank : nullptr);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && to_particles && rebuild_rank && !rank_here) {
        k_rank_of<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->sout, a.n, c->rank);
        e = hipGetLastError();
    }
    if (e == hipSuccess && to_particles) {
        k_scatter<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->sout, c->rank, a.n, c->max_n,
                                                              F.flags, px, py, pz, vx, vy, vz,
                                                              density, accel);
        e = hipGetLastError();
    }
    tend(c, KID_FINAL);
    return e;
}

}  // namespace fh
