// fh_sph_fast.hip -- LDS-tiled SPH density and pressure/viscosity passes for gfx950.
//
// Work decomposition.  A workgroup (256 lanes) owns 256 consecutive particles of the cell-sorted
// order (a "tile") and one z-slab dz in {-1, 0, +1} of their 3x3x3 neighbourhood, so every tile
// is processed by three workgroups whose partial sums land in three separate buffers (summed
// later in a fixed order: results are deterministic, no atomics).  Splitting by slab divides the
// critical path of tiles that sit in very dense cells by three.
//
// Neighbour staging.  For a fixed (dy, dz) the three x-adjacent cells of a particle are one
// contiguous range of the sorted arrays, and because sorted particles have non-decreasing cells
// the union of those ranges over a tile is itself one contiguous range.  Each of the 3 rows of
// the slab is streamed through LDS in 512-particle chunks with coalesced float4 loads; every lane
// then walks only its own sub-range of the chunk, reading LDS (broadcast when lanes share a
// cell, which is the common case in dense regions).  All loop bounds that contain barriers are
// workgroup-uniform.
//
// XCD mapping.  Workgroups are dispatched round-robin over the 8 XCDs; work item ids are
// remapped so each XCD processes one contiguous block of tiles and its L2 holds that region of
// the sorted arrays and its neighbour rows.
//
// Arithmetic.  Same quantities as the reference kernels (sph_density.rs:413-453,
// sph_fused.rs:552-637) with fused multiply-adds, a hardware reciprocal square root for 1/r and
// the pressure and viscosity terms summed into one accumulator; the per-slab partials are added
// as (slab -1 + slab 0) + slab +1.  Differences to the CPU restatement are rounding only
// (checked against rel 1e-4 on density and 1e-4 * sum|pair terms| on accelerations).
#include "fh_internal.hpp"

namespace fh {

constexpr int kTileP = 256;   // home particles per workgroup
constexpr int kStage = 512;   // neighbour particles staged per chunk
constexpr uint32_t kEmpty = 0xFFFFFFFFu;

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

// The three row ranges [b, e) of slab dz for one particle (cells clamped like the reference,
// sph_density.rs:421-437); empty ranges for rows outside the grid.
__device__ __forceinline__ void slab_ranges(const float4& p, bool live, const GridDesc& g,
                                            const uint32_t* __restrict__ cstart, uint32_t n,
                                            int dz, uint32_t b[3], uint32_t e[3]) {
#pragma unroll
    for (int r = 0; r < 3; r++) {
        b[r] = 0u;
        e[r] = 0u;
    }
    if (!live) return;
    const int cx = (int)cell_coord(p.x, 0.0f, g.cs, g.nx);
    const int cy = (int)cell_coord(p.y, 0.0f, g.cs, g.ny);
    const int cz = (int)cell_coord(p.z, 0.0f, g.cs, g.nz);
    const int nz = cz + dz;
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
// is moved to a heavy list and processed by a 1024-lane workgroup in which 16 waves split the
// candidates of the same 64 particles and reduce their partial sums in wave order.  The light
// kernels skip those items.  The plan is made once per substep and serves both passes.
constexpr int kSub = 64;                // particles per sub-tile (one wavefront)
constexpr int kHeavyThreads = 1024;     // 16 waves per heavy workgroup
constexpr int kHeavyWaves = kHeavyThreads / kWave;
constexpr int kHeavyStage = 1024;       // staged candidates per chunk (64 per wave)
constexpr uint32_t kHeavyWork = 1024;   // candidates per particle and slab
constexpr uint32_t kHeavyGrid = 512;    // heavy workgroups (grid-stride over the list)

// Candidate density accumulation of one lane over [jb, je) of a staged chunk, four candidates
// per iteration with independent accumulators so LDS latency and the FMA chain overlap.
__device__ __forceinline__ float density_run(const float4* __restrict__ sp, uint32_t c0,
                                             uint32_t jb, uint32_t je, float4 pi, float h2,
                                             float acc) {
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    uint32_t j = jb;
    for (; j + 4 <= je; j += 4) {
        const float4 q0 = sp[j - c0], q1 = sp[j + 1 - c0], q2 = sp[j + 2 - c0], q3 = sp[j + 3 - c0];
        float dx = pi.x - q0.x, dy = pi.y - q0.y, dz = pi.z - q0.z;
        float d = fmaxf(h2 - fmaf(dz, dz, fmaf(dy, dy, dx * dx)), 0.0f);
        a0 = fmaf(d * d, d, a0);
        dx = pi.x - q1.x; dy = pi.y - q1.y; dz = pi.z - q1.z;
        d = fmaxf(h2 - fmaf(dz, dz, fmaf(dy, dy, dx * dx)), 0.0f);
        a1 = fmaf(d * d, d, a1);
        dx = pi.x - q2.x; dy = pi.y - q2.y; dz = pi.z - q2.z;
        d = fmaxf(h2 - fmaf(dz, dz, fmaf(dy, dy, dx * dx)), 0.0f);
        a2 = fmaf(d * d, d, a2);
        dx = pi.x - q3.x; dy = pi.y - q3.y; dz = pi.z - q3.z;
        d = fmaxf(h2 - fmaf(dz, dz, fmaf(dy, dy, dx * dx)), 0.0f);
        a3 = fmaf(d * d, d, a3);
    }
    for (; j < je; j++) {
        const float4 q = sp[j - c0];
        const float dx = pi.x - q.x, dy = pi.y - q.y, dz = pi.z - q.z;
        const float d = fmaxf(h2 - fmaf(dz, dz, fmaf(dy, dy, dx * dx)), 0.0f);
        a0 = fmaf(d * d, d, a0);
    }
    return acc + ((a0 + a1) + (a2 + a3));
}

// Plan: per (sub-tile, slab) the largest per-particle candidate count decides light / heavy.
__global__ __launch_bounds__(256) void k_plan(const float4* __restrict__ spos, uint32_t n,
                                              GridDesc g, const uint32_t* __restrict__ cstart,
                                              uint8_t* __restrict__ flag,
                                              uint32_t* __restrict__ heavy, Control* ctl) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t sub = s / kSub;
    const bool live = s < n;
    if (sub * kSub >= n) return;  // whole wave beyond the particles
    const float4 pi = live ? spos[s] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int slab = 0; slab < 3; slab++) {
        uint32_t b[3], e[3];
        slab_ranges(pi, live, g, cstart, n, slab - 1, b, e);
        const uint32_t w = wave_max((e[0] - b[0]) + (e[1] - b[1]) + (e[2] - b[2]));
        if ((threadIdx.x & 63) == 0) {
            const uint32_t item = sub * 3u + (uint32_t)slab;
            const bool hv = w > kHeavyWork;
            flag[item] = hv ? 1 : 0;
            if (hv) heavy[atomicAdd(&ctl->heavy_count.v, 1u)] = item;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// The staged chunk sequence of one slab: the union [lo[r], hi[r]) of each of the 3 rows, cut
// into chunks of `ch` candidates, rows in dy order.  Chunks are double-buffered in LDS: chunk
// q + 1 is fetched into registers while chunk q is consumed, so one barrier per chunk suffices
// and global latency overlaps the pair work.
struct ChunkSeq {
    uint32_t lo[3], n[3], total, ch;
    __device__ __forceinline__ ChunkSeq(const uint32_t l[3], const uint32_t h[3], uint32_t c) {
        ch = c;
        total = 0;
#pragma unroll
        for (int r = 0; r < 3; r++) {
            lo[r] = l[r];
            n[r] = l[r] < h[r] ? (h[r] - l[r] + c - 1) / c : 0u;
            total += n[r];
        }
        hi0 = h[0];
        hi1 = h[1];
        hi2 = h[2];
    }
    uint32_t hi0, hi1, hi2;
    // chunk q -> row r, first candidate c0, size m
    __device__ __forceinline__ void at(uint32_t q, int& r, uint32_t& c0, uint32_t& m) const {
        uint32_t hi;
        if (q < n[0]) {
            r = 0;
            c0 = lo[0] + q * ch;
            hi = hi0;
        } else if (q < n[0] + n[1]) {
            r = 1;
            c0 = lo[1] + (q - n[0]) * ch;
            hi = hi1;
        } else {
            r = 2;
            c0 = lo[2] + (q - n[0] - n[1]) * ch;
            hi = hi2;
        }
        m = min(ch, hi - c0);
    }
};

__device__ __forceinline__ uint32_t pick3(const uint32_t v[3], int r) {
    return r == 0 ? v[0] : (r == 1 ? v[1] : v[2]);
}

// Home-row segments.  A wave owns 64 consecutive sorted particles (a sub-tile); the particles of
// one home row (cy, cz) are consecutive lanes, and for each of the slab's 3 rows the union of
// their neighbour ranges is one short contiguous range (x-adjacent cells of that row only).
// The wave walks its segments one at a time and stages each union through its own LDS slice
// 64 candidates at a time: no workgroup barrier anywhere, so waves never wait for each other
// and a sparse sub-tile spanning many rows never stages the unrelated cells between them.
__device__ __forceinline__ uint32_t home_row(const float4& p, const GridDesc& g) {
    return cell_coord(p.y, 0.0f, g.cs, g.ny) + cell_coord(p.z, 0.0f, g.cs, g.nz) * g.ny;
}

// Density partials: dpart[slab][s] = sum over the slab's neighbours j of (h^2 - r^2)^3, r^2 < h^2.
__global__ __launch_bounds__(kTileP) void k_density_wave(const float4* __restrict__ spos,
                                                         uint32_t n, GridDesc g,
                                                         const uint32_t* __restrict__ cstart,
                                                         float h2, float* __restrict__ dpart,
                                                         uint32_t stride, uint32_t items,
                                                         const uint8_t* __restrict__ flag) {
    __shared__ float4 s_p[kTileP / kWave][kWave];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t item = blockIdx.x * (kTileP / kWave) + (uint32_t)wave;
    if (item >= items) return;  // whole wave
    const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
    const uint32_t s = sub * kSub + (uint32_t)lane;
    const bool live = s < n && !flag[item];
    const float4 pi = live ? spos[s] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    uint32_t b[3], e[3];
    slab_ranges(pi, live, g, cstart, n, (int)slab - 1, b, e);
    const uint32_t hr = home_row(pi, g);
    float4* buf = s_p[wave];
    float acc = 0.0f;
    uint64_t pending = __ballot(live);
    while (pending) {  // wave-uniform
        const int leader = __ffsll((unsigned long long)pending) - 1;
        const uint32_t row = (uint32_t)__shfl((int)hr, leader, kWave);
        const bool mine = live && hr == row;
        const uint64_t seg = __ballot(mine);
        pending &= ~seg;
        const int last = 63 - __clzll((long long)seg);
#pragma unroll
        for (int r = 0; r < 3; r++) {
            // the segment's lanes share the home row (so the same valid rows) and have
            // non-decreasing ranges: the union is [b of the first lane, e of the last lane)
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)b[r], leader);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)e[r], last);
            for (uint32_t c0 = lo; c0 < hi; c0 += kWave) {
                const uint32_t m = min((uint32_t)kWave, hi - c0);
                __builtin_amdgcn_wave_barrier();
                buf[lane] = (uint32_t)lane < m ? spos[c0 + lane] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                __builtin_amdgcn_wave_barrier();
                if (mine) acc = density_run(buf, c0, max(b[r], c0), min(e[r], c0 + m), pi, h2, acc);
            }
        }
    }
    if (live) dpart[(size_t)slab * stride + s] = acc;
}

// Heavy items: 16 waves share the 64 particles of one (sub-tile, slab); wave w walks slots
// [64 w, 64 w + 64) of every staged 1024-candidate chunk.
__global__ __launch_bounds__(kHeavyThreads) void k_density_heavy(
    const float4* __restrict__ spos, uint32_t n, GridDesc g, const uint32_t* __restrict__ cstart,
    float h2, float* __restrict__ dpart, uint32_t stride, const uint32_t* __restrict__ heavy,
    const Control* __restrict__ ctl) {
    __shared__ float4 s_p[2][kHeavyStage];
    __shared__ float s_acc[kHeavyWaves][kSub];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t count = ctl->heavy_count.v;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t it = blockIdx.x; it < count; it += gridDim.x) {  // uniform
        const uint32_t item = heavy[it];
        const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
        const uint32_t s = sub * kSub + (uint32_t)lane;
        const bool live = s < n;
        const float4 pi = live ? spos[s] : z4;
        uint32_t b[3], e[3], lo[3], hi[3];
        slab_ranges(pi, live, g, cstart, n, (int)slab - 1, b, e);
#pragma unroll
        for (int q = 0; q < 3; q++) {  // every wave holds the same particles: wave-local unions
            lo[q] = wave_min(b[q] < e[q] ? b[q] : kEmpty);
            hi[q] = wave_max(b[q] < e[q] ? e[q] : 0u);
        }
        const ChunkSeq cq(lo, hi, kHeavyStage);
        int r;
        uint32_t c0, m;
        float4 fa = z4;
        if (cq.total) {
            cq.at(0, r, c0, m);
            if ((uint32_t)tid < m) fa = spos[c0 + tid];
        }
        float acc = 0.0f;
        for (uint32_t q = 0; q < cq.total; q++) {
            float4* buf = s_p[q & 1u];
            buf[tid] = fa;
            __syncthreads();
            if (q + 1 < cq.total) {
                cq.at(q + 1, r, c0, m);
                fa = (uint32_t)tid < m ? spos[c0 + tid] : z4;
            }
            cq.at(q, r, c0, m);
            const uint32_t sb = c0 + (uint32_t)wave * kSub;
            const uint32_t se = min(sb + (uint32_t)kSub, c0 + m);
            const uint32_t jb = max(pick3(b, r), sb), je = min(pick3(e, r), se);
            acc = density_run(buf, c0, jb, je, pi, h2, acc);
        }
        s_acc[wave][lane] = acc;
        __syncthreads();
        if (wave == 0) {
            float t = 0.0f;
            for (int w = 0; w < kHeavyWaves; w++) t += s_acc[w][lane];
            if (live) dpart[(size_t)slab * stride + s] = t;
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
struct FastForce {
    float h, h2, mc, k, rho0;
    float fp;  // -mass * gcoef / 2: pressure pair term = fp*(p_i+p_j)/rho_j*(h-r)^2/r * (x_i-x_j)
    float fv;  // mu * mass * lcoef: viscosity pair term = fv/rho_j*(h-r) * (v_j-v_i)
};

__device__ __forceinline__ float rho_of(const float* __restrict__ dpart, uint32_t stride,
                                        uint32_t j, float mc) {
    return mc * ((dpart[j] + dpart[stride + j]) + dpart[2u * stride + j]);
}

// One prefetched candidate of the force pass: position, velocity and its three density
// partials; converted at store time to (x, y, z, p_j) and (vx, vy, vz, 1/rho_j), where 1/rho_j
// is 0 when rho_j < 1e-6 -- that removes the pair exactly like the skip of sph_fused.rs:607.
struct ForceSlot {
    float4 q, w;
    float d0, d1, d2;
};

__device__ __forceinline__ ForceSlot force_fetch(const float4* __restrict__ spos,
                                                 const float4* __restrict__ svel,
                                                 const float* __restrict__ dpart,
                                                 uint32_t stride, uint32_t j, bool ok) {
    ForceSlot f;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    f.q = ok ? spos[j] : z4;
    f.w = ok ? svel[j] : z4;
    f.d0 = ok ? dpart[j] : 0.0f;
    f.d1 = ok ? dpart[stride + j] : 0.0f;
    f.d2 = ok ? dpart[2u * stride + j] : 0.0f;
    return f;
}

__device__ __forceinline__ void force_store(float4* __restrict__ sp, float4* __restrict__ sv,
                                            uint32_t t, const ForceSlot& f, const FastForce& K) {
    const float rj = K.mc * ((f.d0 + f.d1) + f.d2);
    sp[t] = make_float4(f.q.x, f.q.y, f.q.z, K.k * (rj - K.rho0));
    sv[t] = make_float4(f.w.x, f.w.y, f.w.z, rj < 1e-6f ? 0.0f : 1.0f / rj);
}

// Pressure + viscosity pair terms of one lane over [jb, je) of a staged chunk.
__device__ __forceinline__ void force_run(const float4* __restrict__ sp,
                                          const float4* __restrict__ sv, uint32_t c0,
                                          uint32_t jb, uint32_t je, float4 pi, float4 vi,
                                          float p_i, const FastForce& K, float& ax, float& ay,
                                          float& az) {
#pragma unroll 2
    for (uint32_t j = jb; j < je; j++) {
        const float4 q = sp[j - c0];
        const float dx = pi.x - q.x, dy = pi.y - q.y, dz = pi.z - q.z;
        const float r2 = fmaf(dz, dz, fmaf(dy, dy, dx * dx));
        if (r2 < K.h2 && r2 > 1e-12f) {
            const float4 w = sv[j - c0];
            const float rinv = __builtin_amdgcn_rsqf(r2);
            const float diff = K.h - r2 * rinv;
            const float fs = K.fp * (p_i + q.w) * w.w * (diff * diff) * rinv;
            const float vs = K.fv * w.w * diff;
            ax = fmaf(vs, w.x - vi.x, fmaf(fs, dx, ax));
            ay = fmaf(vs, w.y - vi.y, fmaf(fs, dy, ay));
            az = fmaf(vs, w.z - vi.z, fmaf(fs, dz, az));
        }
    }
}

// Acceleration partials: fpart[slab][c][s] = sum over the slab's neighbours j of the pressure
// and viscosity pair terms (sph_fused.rs:604-623), not yet divided by rho_i.  Same wave-private
// home-row segments as k_density_wave.
__global__ __launch_bounds__(kTileP) void k_force_wave(const float4* __restrict__ spos,
                                                       const float4* __restrict__ svel,
                                                       const float* __restrict__ dpart,
                                                       uint32_t n, GridDesc g,
                                                       const uint32_t* __restrict__ cstart,
                                                       FastForce K, float* __restrict__ fpart,
                                                       uint32_t stride, uint32_t items,
                                                       const uint8_t* __restrict__ flag) {
    __shared__ float4 s_p[kTileP / kWave][kWave];  // x, y, z, p_j
    __shared__ float4 s_v[kTileP / kWave][kWave];  // vx, vy, vz, 1/rho_j
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t item = blockIdx.x * (kTileP / kWave) + (uint32_t)wave;
    if (item >= items) return;
    const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
    const uint32_t s = sub * kSub + (uint32_t)lane;
    const bool in = s < n && !flag[item];  // heavy items: k_force_heavy
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const float4 pi = in ? spos[s] : z4;
    const float4 vi = in ? svel[s] : z4;
    const float rho_i = in ? rho_of(dpart, stride, s, K.mc) : 0.0f;
    const bool live = in && !(rho_i < 1e-6f);  // sph_fused.rs:550
    const float p_i = K.k * (rho_i - K.rho0);
    uint32_t b[3], e[3];
    slab_ranges(pi, live, g, cstart, n, (int)slab - 1, b, e);
    const uint32_t hr = home_row(pi, g);
    float4* bp = s_p[wave];
    float4* bv = s_v[wave];
    float ax = 0.0f, ay = 0.0f, az = 0.0f;
    uint64_t pending = __ballot(live);
    while (pending) {
        const int leader = __ffsll((unsigned long long)pending) - 1;
        const uint32_t row = (uint32_t)__shfl((int)hr, leader, kWave);
        const bool mine = live && hr == row;
        const uint64_t seg = __ballot(mine);
        pending &= ~seg;
        const int last = 63 - __clzll((long long)seg);
#pragma unroll
        for (int r = 0; r < 3; r++) {
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)b[r], leader);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)e[r], last);
            for (uint32_t c0 = lo; c0 < hi; c0 += kWave) {
                const uint32_t m = min((uint32_t)kWave, hi - c0);
                const ForceSlot f = force_fetch(spos, svel, dpart, stride, c0 + lane,
                                                (uint32_t)lane < m);
                __builtin_amdgcn_wave_barrier();
                force_store(bp, bv, lane, f, K);
                __builtin_amdgcn_wave_barrier();
                if (mine)
                    force_run(bp, bv, c0, max(b[r], c0), min(e[r], c0 + m), pi, vi, p_i, K, ax,
                              ay, az);
            }
        }
    }
    if (in) {
        float* o = fpart + (size_t)slab * 3u * stride;
        o[s] = ax;
        o[stride + s] = ay;
        o[2u * (size_t)stride + s] = az;
    }
}

__global__ __launch_bounds__(kHeavyThreads) void k_force_heavy(
    const float4* __restrict__ spos, const float4* __restrict__ svel,
    const float* __restrict__ dpart, uint32_t n, GridDesc g, const uint32_t* __restrict__ cstart,
    FastForce K, float* __restrict__ fpart, uint32_t stride, const uint32_t* __restrict__ heavy,
    const Control* __restrict__ ctl) {
    __shared__ float4 s_p[2][kHeavyStage];
    __shared__ float4 s_v[2][kHeavyStage];
    __shared__ float s_acc[3][kHeavyWaves][kSub];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t count = ctl->heavy_count.v;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (uint32_t it = blockIdx.x; it < count; it += gridDim.x) {  // uniform
        const uint32_t item = heavy[it];
        const uint32_t sub = item / 3u, slab = item - 3u * (item / 3u);
        const uint32_t s = sub * kSub + (uint32_t)lane;
        const bool in = s < n;
        const float4 pi = in ? spos[s] : z4;
        const float4 vi = in ? svel[s] : z4;
        const float rho_i = in ? rho_of(dpart, stride, s, K.mc) : 0.0f;
        const bool live = in && !(rho_i < 1e-6f);
        const float p_i = K.k * (rho_i - K.rho0);
        uint32_t b[3], e[3], lo[3], hi[3];
        slab_ranges(pi, live, g, cstart, n, (int)slab - 1, b, e);
#pragma unroll
        for (int q = 0; q < 3; q++) {
            lo[q] = wave_min(b[q] < e[q] ? b[q] : kEmpty);
            hi[q] = wave_max(b[q] < e[q] ? e[q] : 0u);
        }
        const ChunkSeq cq(lo, hi, kHeavyStage);
        int r;
        uint32_t c0, m;
        ForceSlot fa;
        {
            uint32_t c = 0, mm = 0;
            if (cq.total) cq.at(0, r, c, mm);
            fa = force_fetch(spos, svel, dpart, stride, c + tid, (uint32_t)tid < mm);
        }
        float ax = 0.0f, ay = 0.0f, az = 0.0f;
        for (uint32_t q = 0; q < cq.total; q++) {
            float4* bp = s_p[q & 1u];
            float4* bv = s_v[q & 1u];
            force_store(bp, bv, tid, fa, K);
            __syncthreads();
            if (q + 1 < cq.total) {
                cq.at(q + 1, r, c0, m);
                fa = force_fetch(spos, svel, dpart, stride, c0 + tid, (uint32_t)tid < m);
            }
            cq.at(q, r, c0, m);
            const uint32_t sb = c0 + (uint32_t)wave * kSub;
            const uint32_t se = min(sb + (uint32_t)kSub, c0 + m);
            const uint32_t jb = max(pick3(b, r), sb), je = min(pick3(e, r), se);
            force_run(bp, bv, c0, jb, je, pi, vi, p_i, K, ax, ay, az);
        }
        s_acc[0][wave][lane] = ax;
        s_acc[1][wave][lane] = ay;
        s_acc[2][wave][lane] = az;
        __syncthreads();
        if (wave < 3) {  // wave c reduces component c in wave order
            float t = 0.0f;
            for (int w = 0; w < kHeavyWaves; w++) t += s_acc[wave][w][lane];
            if (in) fpart[((size_t)slab * 3u + (uint32_t)wave) * stride + s] = t;
        }
        __syncthreads();
    }
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
// integrate.rs:23-29, box_collider.rs:37-46), scatter everything back to particle order.
__global__ __launch_bounds__(256) void k_finalize(const float4* __restrict__ spos,
                                                  const float4* __restrict__ svel,
                                                  const float* __restrict__ dpart,
                                                  const float* __restrict__ fpart,
                                                  const uint32_t* __restrict__ sidx, uint32_t n,
                                                  uint32_t stride, Finish F,
                                                  float* __restrict__ px, float* __restrict__ py,
                                                  float* __restrict__ pz, float* __restrict__ vx,
                                                  float* __restrict__ vy, float* __restrict__ vz,
                                                  float* __restrict__ density,
                                                  float* __restrict__ accel) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const uint32_t i = sidx[s];
    if (i >= n) return;
    const float rho = rho_of(dpart, stride, s, F.mc);
    if (density) density[i] = rho;
    if (F.flags & kDensityOnly) return;
    const float4 p = spos[s];
    const float4 v = svel[s];
    float ax = 0.0f, ay = 0.0f, az = 0.0f;
    float nvx = v.x, nvy = v.y, nvz = v.z;
    if (!(rho < 1e-6f)) {
        const float inv = 1.0f / rho;
        const size_t S = stride;
        ax = ((fpart[s] + fpart[3 * S + s]) + fpart[6 * S + s]) * inv;
        ay = ((fpart[S + s] + fpart[4 * S + s]) + fpart[7 * S + s]) * inv;
        az = ((fpart[2 * S + s] + fpart[5 * S + s]) + fpart[8 * S + s]) * inv;
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
    vx[i] = nvx;
    vy[i] = nvy;
    vz[i] = nvz;
    if (F.flags & (FH_EPI_INTEGRATE | FH_EPI_BOX)) {
        px[i] = npx;
        py[i] = npy;
        pz[i] = npz;
    }
    if (accel) {
        accel[i] = ax;
        accel[(size_t)n + i] = ay;
        accel[2 * (size_t)n + i] = az;
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

hipError_t launch_plan(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start) {
    if (a.n == 0) return hipSuccess;
    tbeg(c, KID_PLAN);
    k_plan<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->spos, a.n, a.g, cell_start,
                                                       c->heavy_flag, c->heavy, c->ctl);
    tend(c, KID_PLAN);
    return hipGetLastError();
}

hipError_t launch_density_fast(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start) {
    if (a.n == 0) return hipSuccess;
    uint32_t items;
    const uint32_t grid = wave_grid(a.n, &items);
    tbeg(c, KID_DENSITY);
    k_density_wave<<<grid, kTileP, 0, c->stream>>>(c->spos, a.n, a.g, cell_start, a.h * a.h,
                                                   c->dpart, c->max_n, items, c->heavy_flag);
    tend(c, KID_DENSITY);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    tbeg(c, KID_DHEAVY);
    k_density_heavy<<<kHeavyGrid, kHeavyThreads, 0, c->stream>>>(
        c->spos, a.n, a.g, cell_start, a.h * a.h, c->dpart, c->max_n, c->heavy, c->ctl);
    tend(c, KID_DHEAVY);
    return hipGetLastError();
}

hipError_t launch_force_fast(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start) {
    if (a.n == 0) return hipSuccess;
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
    uint32_t items;
    const uint32_t grid = wave_grid(a.n, &items);
    tbeg(c, KID_FORCE);
    k_force_wave<<<grid, kTileP, 0, c->stream>>>(c->spos, c->svel, c->dpart, a.n, a.g,
                                                 cell_start, K, c->fpart, c->max_n, items,
                                                 c->heavy_flag);
    tend(c, KID_FORCE);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    tbeg(c, KID_FHEAVY);
    k_force_heavy<<<kHeavyGrid, kHeavyThreads, 0, c->stream>>>(
        c->spos, c->svel, c->dpart, a.n, a.g, cell_start, K, c->fpart, c->max_n, c->heavy, c->ctl);
    tend(c, KID_FHEAVY);
    return hipGetLastError();
}

hipError_t launch_finalize(fh_ctx* c, const SphArgs& a, const fh_epilogue* epi, bool density_only,
                           float* px, float* py, float* pz, float* vx, float* vy, float* vz,
                           float* density, float* accel) {
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
    k_finalize<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->spos, c->svel, c->dpart, c->fpart,
                                                           c->sidx, a.n, c->max_n, F, px, py, pz,
                                                           vx, vy, vz, density, accel);
    tend(c, KID_FINAL);
    return hipGetLastError();
}

}  // namespace fh
