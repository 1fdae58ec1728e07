// fh_internal.hpp -- context layout, shared device helpers and launcher declarations of the
// gfx950 SPH / hash-grid library.  Every translation unit of libforge_hip.so includes this.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/forge_hip.h"

namespace fh {

// ---- sizes ----------------------------------------------------------------------------------
constexpr int kWave = 64;              // CDNA wavefront
#ifndef FH_SORT_THREADS
#define FH_SORT_THREADS 512
#endif
#ifndef FH_SORT_ITEMS
#define FH_SORT_ITEMS 16
#endif
#ifndef FH_SORT_MINB
#define FH_SORT_MINB 4  // sort workgroups per CU the register budget is sized for
#endif
constexpr int kSortThreads = FH_SORT_THREADS;  // 8 waves per sort workgroup
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortItems = FH_SORT_ITEMS;      // keys per thread per tile
constexpr int kSortTile = kSortThreads * kSortItems;  // 8192 keys per tile
constexpr int kSortItemsLarge = 24;                  // keys per thread from kSortLargeN keys on
constexpr int kSortTileLarge = kSortThreads * kSortItemsLarge;
constexpr uint32_t kSortLargeN = 1u << 22;
constexpr int kMaxPasses = 4;          // 8-bit digits, up to 32-bit keys
// Digit layouts of a sort.  8-bit digits in general; 10-bit digits for keys of 17..20 bits
// below kWideMaxN keys (c3's and c2's cell keys): two passes instead of three.  A pass over
// that many keys costs about the same at either width -- its time is the look-back chain across
// the tiles, not its bytes -- so the pass saved is the gain (c2's build, 4,194,304 keys of 20
// bits: 0.138 -> 0.124 ms).  10-bit passes always use kSortTile-key tiles.
constexpr uint32_t kWideDigitBits = 10;
constexpr uint32_t kWideMaxN = 1u << 23;
// Words per tile of look-back and per row of partial histograms, and Control::hist: the largest
// passes x bins over the layouts (4 x 256, 2 x 1024).  Pass p's bin d sits at p * bins + d.
constexpr uint32_t kDigitSlots = 2048;
constexpr int kHistThreads = 256;
#ifndef FH_HIST_ITEMS
#define FH_HIST_ITEMS 16
#endif
constexpr int kHistItems = FH_HIST_ITEMS;
constexpr int kHistChunk = kHistThreads * kHistItems;  // keys per histogram chunk
constexpr int kPreItems = kHistChunk / kSortThreads;     // keys per thread of a first pass with prefixes
#ifndef FH_HIST_BLOCKS
#define FH_HIST_BLOCKS 1024
#endif
constexpr int kHistBlocks = FH_HIST_BLOCKS;  // rows of per-block partial histograms
#ifndef FH_HIST_ROWS_PER_REDUCE
#define FH_HIST_ROWS_PER_REDUCE 32
#endif
// Partial rows summed by one reduce workgroup of a small sort, whose first pass adds the sums of
// the groups before its tile (c2's build, 512 two-row tiles: groups of 8 rows took 0.110 ms, 16
// 0.104, 32 0.100, 64 0.0997, 128 0.102; with c3's one-row tiles 32 rows against 64: c3 396.2
// against 397.2 us per substep, c2 0.098 against 0.100 ms)
constexpr int kHistRowsPerReduce = FH_HIST_ROWS_PER_REDUCE;
// A first pass with prefixes runs on tiles of one histogram row (4096 keys: twice the workgroups)
// up to kPreSmallMaxN keys, where the tiles then fill the GPU in about one round (c3: 396.7 against
// 398.7 us per substep, c0 86.7 against 89.5 us), and on tiles of two rows above (c2's 4,194,304
// keys: 0.100 against 0.108 ms with one-row tiles)
constexpr uint32_t kPreSmallMaxN = 1u << 21;
__host__ __device__ inline uint32_t pre_rows_per_tile(uint32_t n) { return n <= kPreSmallMaxN ? 1u : 2u; }
constexpr int kHistRowsPlain = 8;  // rows per reduce workgroup of a sort without first-pass prefixes
constexpr uint32_t kMaxSortN = 1u << 30;  // look-back words hold 30-bit counts
// Co-located particles: when at least kCollapseMin particles of a cell sit at one position (the
// box corners of a dam break collect thousands, next to a few hundred others), the cell is
// reordered so they come first.  The first of them (the representative) stands for the group:
// as a home particle it is computed once for all, as a neighbour it is one candidate of weight
// M carrying the summed velocity of the group.  spos[s].w holds raw bits: s for an ordinary
// particle, M | kRepFlag for a representative, the representative's index for the others.
constexpr uint32_t kCollapseMin = 64;
constexpr uint32_t kRepFlag = 0x80000000u;
// A cell of >= kCollapseMin particles is examined in full only when at least kGroupHits of
// kGroupSamples evenly spaced particles sit at the position of one of them (groups that are a
// small minority of their cell are not collapsed; results are the same either way).
constexpr uint32_t kGroupSamples = 16;
constexpr uint32_t kGroupHits = 4;
// The heavy SPH work list is split into kHeavyLists sub-lists with counters on separate lines,
// so that appends from different workgroups do not serialise on one address.
constexpr int kHeavyLists = 8;
#ifndef FH_HW
#define FH_HW 4
#endif
// single-wave parts of a heavy SPH item: kHeavyWaves by default, kHeavyWavesMax with
// FH_OPT_HEAVY_PARTS or for small systems (the partial-sum slots then have room for it)
constexpr int kHeavyWaves = FH_HW, kHeavyWavesMax = 8;
// Systems of fewer particles have too few (sub-tile, slab) items to fill the GPU (configs[0]'s
// 50,000: 2,346 items for 1,024 SIMDs): by default the fast passes split more of their items,
// into kHeavyWavesMax parts (contexts of smaller max_n make room for them at creation).
constexpr uint32_t kSmallSystemN = 1u << 18;
constexpr int kHeavyComps = 4;      // partial sums per lane and part: a_x, a_y, a_z, w (density: 1)
// A light item's candidate stream as the plan or the density pass leaves it for the passes: per
// lane, its three row starts and three counts in the stream (10 bits each, two words), then the
// sorted indices of the first two windows' staging slots (256 each) as 16-bit offsets from a
// base at or below the stream's lowest index (two per word).  Streams longer than two windows,
// or spanning more than 65,536 sorted slots, are rebuilt by each pass.
constexpr uint32_t kLightCacheWords = 2 * 64 + 256;
#ifndef FH_PLAN_THREADS
#define FH_PLAN_THREADS 512
#endif
// k_group_plan workgroup: a co-located group, or 8 sub-tiles = 24 (sub-tile, slab) items
constexpr int kPlanThreads = FH_PLAN_THREADS;
constexpr int kEvents = 16;

// The sort's look-back words are 32-bit, [31:30] status, [29:0] value, zeroed by k_begin at
// the start of each sort (half the bytes per poll of a 64-bit word, which is what the walk is
// bound by).  Work tags (co-located groups, skipped sub-tiles, candidate group cells) carry a
// 30-bit epoch that every start bumps; the context renews it before it wraps.
constexpr uint32_t kLb32Aggregate = 1u << 30;
constexpr uint32_t kLb32Inclusive = 2u << 30;
constexpr uint32_t kEpochMask = 0x3FFFFFFFu;
// Bound on look-back polls before a tile gives up and raises the device error flag; keeps
// every wave finite even if an invariant were broken (each poll sleeps ~64 clocks).
constexpr uint32_t kSpinLimit = 1u << 22;

// Device-side control block (one per context).  Every word that is the target of atomics from
// many workgroups sits alone on its own 128-byte line: a line under atomic traffic that also
// holds data every workgroup reads slows those reads down by tens of microseconds per kernel.
struct Line {
    uint32_t v;
    uint32_t pad[31];
};
struct Control {
    uint32_t epoch;                     // bumped by k_begin before each sort / scan
    uint32_t plan;                      // bit p: sort pass p runs (written by pass 0)
    uint32_t spin_limit;                // look-back polls before giving up (0: kSpinLimit)
    uint32_t pad0[29];
    Line error;                         // nonzero: a look-back spin limit was hit
    Line tile_ctr[kMaxPasses];          // dynamic tile ids of the sort passes
    Line scan_ctr;                      // dynamic tile id of the cell scan
    Line heavy_count[kHeavyLists];      // entries in each heavy SPH work sub-list
    Line collapse_count;                // entries in the list of co-located cells
    Line big_count;                     // entries in the list of cells of >= kCollapseMin
    Line triv;                          // bit p: one digit of sort pass p holds all n keys
    uint32_t hist[kDigitSlots];         // digit histograms of the current sort (pass p, bin d: p * bins + d)
};

// Division of a 32-bit unsigned value by a fixed divisor d >= 1 with a multiply-high, a
// subtract, an add and two shifts (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, Figure 4.1): with l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, t = mulhi(m, x), x / d = (t + ((x - t) >> s1)) >> s2
// where (s1, s2) = (min(l, 1), max(l - 1, 0)).  Exact for every x < 2^32.
struct DivU32 {
    uint32_t m, s1, s2;
};

struct GridDesc {
    float cs;
    float ox, oy, oz;
    uint32_t nx, ny, nz;
    DivU32 div_x;   // by nx
    DivU32 div_xy;  // by nx * ny
    uint32_t sb;    // sub-cell bits below the cell in the fast SPH path's sort keys (0, 3, 6, 9)
};

inline DivU32 make_divu32(uint32_t d) {
    uint32_t l = 0;
    while (l < 32 && (1ull << l) < d) l++;
    DivU32 r;
    r.m = (uint32_t)((((1ull << l) - d) << 32) / d + 1);
    r.s1 = l < 1 ? l : 1;
    r.s2 = l > 1 ? l - 1 : 0;
    return r;
}

// Kernels that can be timed with fh_time_kernel (names in kKernelNames).
enum KernelId { KID_HIST, KID_HASH, KID_SCAN, KID_SORT, KID_GATHER, KID_DENSITY,
                KID_FORCE, KID_NBR, KID_FINAL, KID_PLAN, KID_PREP, KID_DPASS,
                KID_FPASS, KID_EPOCH, KID_COUNT };

// Event pairs bracketing the first `max` launches of one kernel after it was armed; when the
// launches are captured, every replay of the graph re-records the same events.
struct Timer {
    uint32_t max, used;
    hipEvent_t* ev;  // 2 * max events
};

}  // namespace fh

struct fh_ctx {
    int device;
    hipStream_t stream;
    bool own_stream;
    uint32_t max_n, max_cells;
    uint32_t max_sort_tiles;
    // sort scratch
    uint32_t* ka;        // [max_n]
    uint32_t* va;        // [max_n]
    uint32_t* kb;        // [max_n]
    uint32_t* vb;        // [max_n]
    uint32_t* sort_lb;   // [max_sort_tiles * kDigitSlots] 32-bit look-back words (pass-major)
    uint32_t* hist_part; // [kHistBlocks][kDigitSlots] per-block digit histograms
    uint32_t* sort_pre;  // first-pass tile prefixes of small sorts (tiles of pre_rows_per_tile
                         // histogram rows): [tiles][1024] within groups of kHistRowsPerReduce rows,
                         // then the groups' sums
                         // (null: the first pass looks back like the others)
    fh::Control* ctl;    // device control block
    // grid scratch
    uint64_t* run_tag;     // [max_cells] epoch << 32: the cell may hold a co-located group
                           // (k_cell_starts' candidates, read by the plan)
    uint32_t* cell_start;  // [max_cells + 1]
    uint32_t* skeys;       // [max_n] sorted keys (cells)
    uint32_t* sidx;        // [max_n] sorted particle ids
    // SPH scratch (sorted order)
    float4* spos;        // [max_n] x, y, z, 0
    float4* svel;        // [max_n] vx, vy, vz, 0
    float* srho;         // [max_n] density (exact kernels; fast force pass via k_prep)
    float* dpart;        // [3][max_n] per-slab density partials (fast kernels)
    float* fpart;        // [3][3][max_n] per-slab acceleration partials (fast kernels)
    uint32_t* heavy;     // [kHeavyLists][heavy_cap] heavy (64-particle tile, slab) work items
    uint32_t heavy_cap;  // entries per heavy sub-list
    uint8_t* heavy_flag; // [3 * ceil(max_n / 64)] 1: heavy list, 2: co-located, skipped
    float* hpart;        // heavy work partials: per slot, hpart_parts x 4 x 64 floats
    uint32_t hpart_parts; // parts per slot the buffer has room for (kHeavyWaves until 8 are asked for)
    uint32_t hslot_cap;  // partial-sum slots in hpart (FH_OPT_HEAVY_SLOTS; default: every item)
    uint32_t* hslot;     // [3 * ceil(max_n / 64)] partial-sum slot of each heavy item, or kNoSlot
    uint32_t* lstream;   // [3 * ceil(max_n / 64)][kLightCacheWords] light items' candidate streams
                         // (lane intervals and window indices) from the density pass, reused by
                         // the force pass
    uint2* lstream_t;    // [3 * ceil(max_n / 64)] stream length of each light item and its lowest
                         // sorted index (~0u: the stream is not kept)
    uint64_t* cell_grp;  // [max_cells] epoch << 32 | number of co-located leading particles
    uint2* big;          // [ceil(max_n / 64) + 1] (first slot, sample offset) of group cells
    uint32_t* skip_tag;  // [ceil(max_n / 64)] epoch of the rebuild whose sub-tile holds only group members
    float* wpart;        // [3][max_n] per-slab viscosity weight sums of representatives (the
                         // planes of dpart, free once k_prep has read them)
    float4* vrep;        // [max_n] summed velocity of the group, at representative indices
    uint32_t* rank;      // [max_n] sorted position of each particle (inverse of sidx)
    uint32_t* sidx2;     // [max_n] resident substeps: previous slot of each new slot
    float4* sout;        // [3 * max_n] new state in sorted order before it is moved to particle
                         // order: pairs (x, y, z, rho), (vx, vy, vz, particle id), then
                         // (ax, ay, az, .); the next substep's input in resident substeps
    bool sph_exact;      // FH_OPT_SPH_EXACT
    uint32_t heavy_work; // FH_OPT_HEAVY_WORK (0: default)
    uint32_t direct_mode; // FH_OPT_DIRECT_ITEMS: 0 never, 1 automatic (default), 2 always
    uint32_t heavy_parts; // FH_OPT_HEAVY_PARTS (0: kHeavyWaves)
    uint32_t sub_bits;    // FH_OPT_SUBCELL: sub-cell key bits of the fused module's fast rebuilds
    uint32_t* h_error;   // pinned host word for the device error flag
    // Epoch renewal.  Tags compare 30-bit epochs, so a tag left 2^30 - 1 starts ago would match
    // again; the host counts the starts it queues (graph replays included) and, before the
    // count reaches epoch_period, queues k_epoch_reset (tags cleared, epoch back to 0).
    uint32_t epoch_period;   // 0: no renewal (the no-alloc sort, which reads no tags)
    uint64_t begins;         // starts queued since the last renewal
    uint32_t capture_begins; // starts recorded by the capture in progress
    uint32_t graph_begins;   // starts per replay of the instantiated graph
    size_t scratch_bytes;
    hipGraph_t graph;
    hipGraphExec_t exec;
    bool capturing;
    hipEvent_t ev[fh::kEvents];
    fh::Timer timers[fh::KID_COUNT];
};

namespace fh {

// ---- shared device helpers -------------------------------------------------------------------

// Cell coordinate along one axis: floor((p - o) / cs) with Rust `as i32` semantics (NaN -> 0,
// saturating) followed by the clamp to [0, dim - 1] (hashgrid.rs:129-136).  The comparisons
// run in float so NaN, +-inf and huge values never reach the float->int conversion.  The
// division is IEEE correctly rounded (the library is built without fast-math), so keys are
// bit-identical to the CPU definition.  Requires dim <= 2^24 (checked on the host).
__device__ __forceinline__ uint32_t cell_coord(float p, float o, float cs, uint32_t dim) {
    float f = floorf((p - o) / cs);
    if (!(f >= 0.0f)) return 0u;
    float top = (float)(dim - 1u);
    if (f >= top) return dim - 1u;
    return (uint32_t)f;
}

__device__ __forceinline__ uint32_t cell_of(float x, float y, float z, const GridDesc& g) {
    uint32_t cx = cell_coord(x, g.ox, g.cs, g.nx);
    uint32_t cy = cell_coord(y, g.oy, g.cs, g.ny);
    uint32_t cz = cell_coord(z, g.oz, g.cs, g.nz);
    return cx + cy * g.nx + cz * g.nx * g.ny;
}

// Sort key of the fast SPH path: the cell, then (g.sb = 3, 6 or 9) the position's sub-cell,
// B = 2, 4 or 8 per axis, in Morton order, so that the particles of a cell lie in compact runs and a
// chunk of consecutive candidates covers a small box.  g.sb = 0: the cell (cell_of).  Positions
// outside the grid keep their clamped cell and a sub-cell clamped to 0..B-1.
__device__ __forceinline__ uint32_t sub_coord(float p, float o, float cs, uint32_t B) {
    const float f = (p - o) / cs;
    const float t = (f - floorf(f)) * (float)B;
    if (!(t >= 0.0f)) return 0u;
    return t >= (float)(B - 1u) ? B - 1u : (uint32_t)t;
}
__device__ __forceinline__ uint32_t sort_key_of(float x, float y, float z, const GridDesc& g) {
    const uint32_t cell = cell_of(x, y, z, g);
    if (g.sb == 0u) return cell;
    const uint32_t B = 1u << (g.sb / 3u);
    const uint32_t sx = sub_coord(x, g.ox, g.cs, B), sy = sub_coord(y, g.oy, g.cs, B),
                   sz = sub_coord(z, g.oz, g.cs, B);
    // interleave: bit b of each coordinate goes to bits 3b, 3b + 1, 3b + 2
    uint32_t m = 0u;
    for (uint32_t b = 0; b < g.sb / 3u; b++)
        m |= (((sx >> b) & 1u) | (((sy >> b) & 1u) << 1) | (((sz >> b) & 1u) << 2)) << (3u * b);
    return (cell << g.sb) | m;
}

__device__ __forceinline__ uint32_t divu32(uint32_t x, DivU32 d) {
    const uint32_t t = __umulhi(d.m, x);
    return (t + ((x - t) >> d.s1)) >> d.s2;
}

// Cell coordinates of a cell key (key = cx + cy * nx + cz * nx * ny, key < nx * ny * nz): the
// exact inverse of cell_of's linearisation, without the float division.
struct CellXYZ {
    int x, y, z;
};
__device__ __forceinline__ CellXYZ key_xyz(uint32_t key, const GridDesc& g) {
    const uint32_t cz = divu32(key, g.div_xy);
    const uint32_t rem = key - cz * (g.nx * g.ny);
    const uint32_t cy = divu32(rem, g.div_x);
    CellXYZ c;
    c.x = (int)(rem - cy * g.nx);
    c.y = (int)cy;
    c.z = (int)cz;
    return c;
}


// Inclusive scan of one value per thread across a 64-lane wavefront.
__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v, int lane) {
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        uint32_t t = __shfl_up(v, off, kWave);
        if (lane >= off) v += t;
    }
    return v;
}

// Exclusive scan of one value per thread over a workgroup of NW waves; `sm` holds NW words.
// Returns the exclusive prefix; *total receives the workgroup sum.  Contains barriers: call
// from uniform control flow only.
template <int NW>
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* sm,
                                                         uint32_t* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t inc = wave_inclusive_scan(v, lane);
    if (lane == 63) sm[wave] = inc;
    __syncthreads();
    uint32_t before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        const uint32_t x = sm[w];
        if (w < wave) before += x;
        sum += x;
    }
    *total = sum;
    __syncthreads();
    return before + inc - v;
}
__device__ __forceinline__ uint32_t block256_exclusive_scan(uint32_t v, uint32_t* sm,
                                                            uint32_t* total) {
    return block_exclusive_scan<4>(v, sm, total);
}

// Bracket a launch with the armed timer's events (no-op when the kernel is not armed).
inline void tbeg(fh_ctx* c, KernelId k, hipStream_t s = nullptr) {
    Timer& t = c->timers[k];
    if (t.used < t.max) (void)hipEventRecord(t.ev[2 * t.used], s ? s : c->stream);
}
inline void tend(fh_ctx* c, KernelId k, hipStream_t s = nullptr) {
    Timer& t = c->timers[k];
    if (t.used < t.max) {
        (void)hipEventRecord(t.ev[2 * t.used + 1], s ? s : c->stream);
        t.used++;
    }
}

// Sets the thread-local message fh_last_error() returns; returns `code`.
int set_error(int code, const char* fmt, ...);
// Account for one start of a sort / rebuild about to be queued (renews the epoch when due).
hipError_t note_begin(fh_ctx* c);
// Default renewal period: every tag epoch stays below the 30-bit wrap.
constexpr uint32_t kEpochPeriod = kEpochMask - 1u;

// ---- launchers (host side, enqueue on ctx->stream; return hipError_t) ------------------------

// Digit histograms of all passes of a num_bits sort of a key array (per-block partials, then
// the reduce).  begin = true also starts a sort (or rebuild): bumps the epoch, clears the
// histograms and counters, and zeroes the look-back words of the coming passes.
hipError_t launch_hist_keys(fh_ctx* c, const uint32_t* keys, uint32_t n, uint32_t num_bits,
                            bool begin);
// Hash particle positions: keys_out[i] = cell, vals_out[i] = i (if non-null) and, for
// num_bits > 0, the digit histograms of all passes of a num_bits sort; begin as above.
hipError_t launch_hash_hist(fh_ctx* c, const float* x, const float* y, const float* z,
                            uint32_t stride, uint32_t n, const GridDesc& g, uint32_t num_bits,
                            uint32_t* keys_out, uint32_t* vals_out, bool begin);
// Run a sort whose histograms are ready: reads (k0, v0) (v0 == nullptr: values are the indices
// 0..n-1), leaves the result in (kfin, vfin).  Either entirely in place ((kfin, vfin) ==
// (k0, v0)) or entirely out of place (kfin may then be null: values only); anything else
// returns hipErrorInvalidValue.  Passes whose digit is the same for every key are skipped on
// the device; the others ping-pong through the context's scratch.
hipError_t launch_sort_passes(fh_ctx* c, const uint32_t* k0, const uint32_t* v0, uint32_t* kfin,
                              uint32_t* vfin, uint32_t n, uint32_t num_bits,
                              uint32_t* rank = nullptr, uint32_t kshift = 0);
hipError_t launch_fill_u32(fh_ctx* c, uint32_t* p, uint32_t value, uint32_t n);
hipError_t launch_boundaries(fh_ctx* c, const uint32_t* sorted_keys, uint32_t n,
                             uint32_t num_cells, uint32_t* cell_start, uint32_t* cell_end);
hipError_t launch_neighbor_query(fh_ctx* c, const float* x, const float* y, const float* z,
                                 uint32_t stride, uint32_t n, const GridDesc& g,
                                 const uint32_t* cell_start, const uint32_t* sorted_indices,
                                 float radius, uint32_t* counts, float* wsum);
hipError_t launch_query(fh_ctx* c, const float* x, const float* y, const float* z,
                        uint32_t stride, const GridDesc& g, const uint32_t* cell_start,
                        const uint32_t* sorted_indices, const float* qx, const float* qy,
                        const float* qz, uint32_t qstride, uint32_t nq, float radius,
                        uint32_t* counts, const uint32_t* offsets, uint32_t* indices);
// SPH passes over the sorted state held in the context.
struct SphArgs {
    GridDesc g;
    float h, mass, k, rho0, mu, dt;
    uint32_t n;
};
// Gather positions (and velocities) into sorted float4 order and mark the key runs.
hipError_t launch_gather(fh_ctx* c, const GridDesc& g, uint32_t cells, const float* px,
                         const float* py, const float* pz, const float* vx, const float* vy,
                         const float* vz, uint32_t n, bool with_vel, bool list_big);
// Resident substeps: the same from the previous substep's sorted state (c->sout), whose slots
// the sort of its keys took as values (sorted: c->sidx2, the previous slot of each new slot).
// The particle ids travel in svel[.].w; c->sidx and c->rank are not maintained (launch_finalize
// rebuilds c->rank from the ids before the final move to particle order).
hipError_t launch_gather_resident(fh_ctx* c, uint32_t cells, uint32_t n);
hipError_t launch_gather_grid(fh_ctx* c, const float* px, const float* py, const float* pz,
                              const float* vx, const float* vy, const float* vz,
                              const float* density, const uint32_t* sorted_indices, uint32_t n);
hipError_t launch_csr_from_sorted(fh_ctx* c, const uint32_t* keys, uint32_t n, uint32_t cells,
                                  uint32_t* cell_start);
hipError_t launch_pack_frame(fh_ctx* c, const float* px, const float* py, const float* pz,
                             uint32_t n, uint32_t frame, uint32_t* counter, void* out);
hipError_t launch_density_fast(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start);
hipError_t launch_force_fast(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start);
// Force records of every sorted particle (positions with pressure, velocity and weight over
// density; density in srho) from the density partials; written into c->sout, which holds the
// new state only after the force pass.
hipError_t launch_prep(fh_ctx* c, const SphArgs& a);
// Fast passes only, one launch: in the cells listed by k_cell_starts, move the particles that
// share the matched sample's position to the front of the cell when they are at least
// kCollapseMin (cell_grp; reorders spos / svel / sidx / rank inside those cells), beside the
// work plan of the fast passes.
hipError_t launch_group_plan(fh_ctx* c, const SphArgs& a, bool with_vel);
// New state in sorted order (c->sout); with `to_particles`, also moved to the caller's arrays
// (`rebuild_rank`: first recompute c->rank from the particle ids, after resident substeps).
// `next_keys` (may be null) receives the cell of each new position, the keys of the next
// resident substep.
hipError_t launch_finalize(fh_ctx* c, const SphArgs& a, const fh_epilogue* epi,
                           bool density_only, float* px, float* py, float* pz, float* vx,
                           float* vy, float* vz, float* density, float* accel,
                           bool to_particles = true, bool rebuild_rank = false,
                           uint32_t* next_keys = nullptr);
hipError_t launch_density(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start,
                          float* density_out);
hipError_t launch_force(fh_ctx* c, const SphArgs& a, const fh_epilogue* epi,
                        const uint32_t* cell_start, float* px, float* py, float* pz, float* vx,
                        float* vy, float* vz, float* accel);
// Unfused pressure (viscosity = false) or viscosity pass over a caller grid, updating v in place
// (the viscosity pass first copies v into c->svel: every neighbour reads the state before it).
hipError_t launch_unfused(fh_ctx* c, bool viscosity, const SphArgs& a, const float* px,
                          const float* py, const float* pz, float* vx, float* vy, float* vz,
                          const float* density, const uint32_t* cell_start,
                          const uint32_t* sorted_indices);
// Copy c->cell_start[0..cells] and c->sidx[0..n) to caller arrays (either may be null).
hipError_t launch_copy_grid(fh_ctx* c, uint32_t cells, uint32_t n, uint32_t* cell_start,
                            uint32_t* sorted_indices);
hipError_t launch_gravity(fh_ctx* c, float* vx, float* vy, float* vz, uint32_t n, float gx,
                          float gy, float gz, float dt);
hipError_t launch_integrate(fh_ctx* c, float* px, float* py, float* pz, float* vx, float* vy,
                            float* vz, uint32_t n, float dt);
hipError_t launch_box(fh_ctx* c, float* px, float* py, float* pz, float* vx, float* vy,
                      float* vz, uint32_t n, const float* mn, const float* mx, float e);

// Digit width, passes and width of the last pass's digit of a num_bits sort of n keys.
struct Digits {
    uint32_t bits, passes, top_bits;
};
__host__ __device__ inline Digits digits_for(uint32_t num_bits, uint32_t n) {
    Digits d;
    d.bits = (num_bits > 16u && num_bits <= 20u && n < kWideMaxN) ? kWideDigitBits : 8u;
    d.passes = (num_bits + d.bits - 1u) / d.bits;
    d.top_bits = num_bits - d.bits * (d.passes ? d.passes - 1u : 0u);
    return d;
}
inline uint32_t bits_for_cells(uint32_t num_cells) {
    uint32_t b = 1;
    while (b < 32 && (1ull << b) < (uint64_t)num_cells) b++;
    return b;
}
__host__ __device__ inline uint32_t ceil_div(uint32_t a, uint32_t b) { return (a + b - 1u) / b; }

}  // namespace fh
