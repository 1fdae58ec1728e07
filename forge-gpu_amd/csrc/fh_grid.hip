// fh_grid.hip -- cell ranges and the 3x3x3 neighbour query for gfx950.  (The CSR cell_start
// of HashGrid::build comes from the sorted keys directly, k_csr_from_sorted in fh_sph.hip.)
//
//   k_fill_u32 +   find_cell_boundaries (radix_sort.rs:229-317): sentinel fill, then one
//   k_boundaries   thread per sorted key marks the first / last index of its run.
//   k_nbr_stream   HashGrid::query_neighbors (hashgrid.rs:145-193) for every point of a built
//                  grid: the 3 x-adjacent cells of one (dy, dz) row are contiguous in the
//                  sorted order, so the 27-cell walk is 9 contiguous ranges visited in the
//                  reference's dz, dy, dx order.
#include "fh_internal.hpp"
#include "fh_stream.hpp"

namespace fh {

// ---------------------------------------------------------------------------------------------
__global__ void k_fill_u32(uint32_t* __restrict__ p, uint32_t value, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = value;
}

hipError_t launch_fill_u32(fh_ctx* c, uint32_t* p, uint32_t value, uint32_t n) {
    if (n == 0) return hipSuccess;
    k_fill_u32<<<ceil_div(n, 256u), 256, 0, c->stream>>>(p, value, n);
    return hipGetLastError();
}

// radix_sort.rs:451-465
__global__ void k_boundaries(const uint32_t* __restrict__ keys, uint32_t n, uint32_t C,
                             uint32_t* __restrict__ cell_start, uint32_t* __restrict__ cell_end) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    uint32_t cell = keys[i];
    if (cell >= C) return;
    if (i == 0 || keys[i - 1] != cell) cell_start[cell] = i;
    if (i == n - 1 || keys[i + 1] != cell) cell_end[cell] = i + 1;
}

hipError_t launch_boundaries(fh_ctx* c, const uint32_t* sorted_keys, uint32_t n,
                             uint32_t num_cells, uint32_t* cell_start, uint32_t* cell_end) {
    hipError_t e = launch_fill_u32(c, cell_start, 0xFFFFFFFFu, num_cells);
    if (e != hipSuccess) return e;
    e = launch_fill_u32(c, cell_end, 0u, num_cells);
    if (e != hipSuccess || n == 0) return e;
    k_boundaries<<<ceil_div(n, 256u), 256, 0, c->stream>>>(sorted_keys, n, num_cells, cell_start,
                                                           cell_end);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Rust `f32 as i32` of an already floored value (NaN -> 0, saturating).
__device__ __forceinline__ int32_t rust_as_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

// The point positions in sorted order (float4), so the query walks contiguous memory.  A
// gather through sorted_indices from the caller's three arrays would read three scattered
// words per point (a cache line each), and a scatter to the sorted slots (through the inverse
// permutation) writes partial cache lines twice (rank, then the float4); instead the points are
// packed once as float4 in their own order (k_pack_pos: coalesced reads and writes), and every
// sorted slot then reads one 16-byte record (k_gather_pos: coalesced sidx reads and writes, one
// scattered 16-byte read per point, mostly served from the MALL, which holds the packed copy).
__global__ __launch_bounds__(256) void k_pack_pos(const float* __restrict__ x,
                                                  const float* __restrict__ y,
                                                  const float* __restrict__ z, uint32_t stride,
                                                  uint32_t n, float4* __restrict__ packed) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const size_t o = (size_t)i * stride;
    packed[i] = make_float4(x[o], y[o], z[o], 0.0f);
}

__global__ __launch_bounds__(256) void k_gather_pos(const float4* __restrict__ packed,
                                                    const uint32_t* __restrict__ sidx,
                                                    uint32_t n, float4* __restrict__ spos) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const uint32_t i = sidx[s];
    // a grid built over these n points holds a permutation of 0..n-1
    spos[s] = i < n ? packed[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// HashGrid::query_neighbors for every point of a built grid, with the neighbour candidates of 64
// consecutive sorted points staged through LDS (the wave candidate stream of fh_stream.hpp, one
// z-slab at a time, kQueryWin candidates per window: a slab's stream of uniform points, ~240
// candidates, mostly fits one window, so a lane's rows are rarely cut by a window edge and the
// row loops, which run as long as their longest lane, run once per slab).  Arithmetic is exactly
// the reference's (the library is built with -ffp-contract=off): diff = p_j - q, dist_sq =
// (dx*dx + dy*dy) + dz*dz, `<=` against radius*radius, weight coeff*diff*diff*diff summed in
// visiting order; each lane visits its own candidates in the reference's order (dz, dy, then
// ascending sorted index), so counts and weight sums are bit-identical to the CPU restatement.
// Points whose query cell lies outside the grid (the reference does not clamp it) take a
// per-lane walk around that cell afterwards.
#ifndef FH_QWIN
#define FH_QWIN 320
#endif
constexpr int kQueryWin = FH_QWIN;

// One candidate: a candidate beyond the radius adds 0 to the count and +0.0f to the weight sum,
// which starts at +0 and only grows, so w + 0.0f == w bit for bit and the sum over the
// candidates is the reference's sum over its neighbours.
__device__ __forceinline__ void nbr_pair(const float4& p, const float4& q, float radius_sq,
                                         float coeff, uint32_t& cnt, float& w) {
    const float dx = p.x - q.x, dy = p.y - q.y, dz = p.z - q.z;
    const float dist_sq = dx * dx + dy * dy + dz * dz;
    const bool ok = dist_sq <= radius_sq;
    const float diff = radius_sq - dist_sq;
    const float t = coeff * diff * diff * diff;
    cnt += ok ? 1u : 0u;
    w += ok ? t : 0.0f;
}

__global__ __launch_bounds__(kWave) void k_nbr_stream(const float4* __restrict__ spos,
                                                      const uint32_t* __restrict__ sidx,
                                                      uint32_t n, GridDesc g,
                                                      const uint32_t* __restrict__ cell_start,
                                                      float radius_sq, float coeff,
                                                      uint32_t* __restrict__ counts,
                                                      float* __restrict__ wsum) {
    constexpr int kLoads = kQueryWin / kWave;
    __shared__ float4 s_p[kQueryWin];
    const int lane = threadIdx.x;
    // runs of consecutive sub-tiles on one XCD: neighbouring sub-tiles read mostly the same
    // candidate rows, which then stay in that XCD's L2
    const uint32_t s = xcd_chunked(blockIdx.x, gridDim.x) * kWave + (uint32_t)lane;
    const bool in = s < n;
    const float4 q = spos[in ? s : 0u];
    // the sort's (clamped) cell, and the reference's unclamped query cell
    const uint32_t cxc = cell_coord(q.x, g.ox, g.cs, g.nx);
    const uint32_t cyc = cell_coord(q.y, g.oy, g.cs, g.ny);
    const uint32_t czc = cell_coord(q.z, g.oz, g.cs, g.nz);
    const int64_t cxu = rust_as_i32(floorf((q.x - g.ox) / g.cs));
    const int64_t cyu = rust_as_i32(floorf((q.y - g.oy) / g.cs));
    const int64_t czu = rust_as_i32(floorf((q.z - g.oz) / g.cs));
    const bool inside = cxu == (int64_t)cxc && cyu == (int64_t)cyc && czu == (int64_t)czc;
    const uint32_t hr = cyc + czc * g.ny;  // home row of the sorted order
    const uint32_t x0 = cxc > 0u ? cxc - 1u : 0u;
    const uint32_t x1 = cxc + 1u < g.nx ? cxc + 1u : g.nx - 1u;
    uint32_t cnt = 0;
    float w = 0.0f;
    for (int dz = -1; dz <= 1; dz++) {  // uniform
        uint32_t b[3], e[3];
        const int nz = (int)czc + dz;
#pragma unroll
        for (int r = 0; r < 3; r++) {
            const int ny = (int)cyc + r - 1;
            b[r] = e[r] = 0u;
            if (in && nz >= 0 && nz < (int)g.nz && ny >= 0 && ny < (int)g.ny) {
                const uint32_t row = (uint32_t)ny * g.nx + (uint32_t)nz * g.nx * g.ny;
                b[r] = cell_start[row + x0];
                e[r] = min(cell_start[row + x1 + 1u], n);
            }
        }
        // a segment's row union runs from its first lane's begin to its last lane's end, which
        // holds because the lanes' clamped ranges grow along the row; an outside point keeps its
        // clamped ranges for the union and evaluates none of them (it is walked later)
        LightStream L;
        light_stream(L, b, e, hr, in, lane);
        if (!inside) {
#pragma unroll
            for (int r = 0; r < 3; r++) L.cnt[r] = 0u;
        }
        for (uint32_t w0 = 0; w0 < L.T; w0 += kQueryWin) {  // uniform
            uint32_t j[kLoads];
            window_indices<kQueryWin>(L, w0, lane, j);
            float4 v[kLoads];
#pragma unroll
            for (int k = 0; k < kLoads; k++) v[k] = spos[j[k]];
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int k = 0; k < kLoads; k++) s_p[k * kWave + lane] = v[k];
            __builtin_amdgcn_wave_barrier();
            // the rows in the reference's dy order (walking them longest first would change
            // the order of the weight sum)
#pragma unroll
            for (int r = 0; r < 3; r++) {
                const uint32_t jb = max(L.S[r], w0);
                const uint32_t je = min(L.S[r] + L.cnt[r], w0 + (uint32_t)kQueryWin);
                // two candidates per step of the LDS address
                // (the bounds are formed from the count, never before the buffer: an address
                // below the LDS buffer's start would wrap around in 32-bit LDS addressing)
                const uint32_t m = je > jb ? je - jb : 0u;
                const float4* c = s_p + (jb - w0);
                const float4* const ce = c + m;
                const float4* const cu = c + (m > 1u ? m - 1u : 0u);
                if (c < cu) {
                    do {
                        const float4 p0 = c[0], p1 = c[1];
                        nbr_pair(p0, q, radius_sq, coeff, cnt, w);
                        nbr_pair(p1, q, radius_sq, coeff, cnt, w);
                        c += 2;
                    } while (c < cu);
                }
                if (c < ce) nbr_pair(*c, q, radius_sq, coeff, cnt, w);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    if (in && !inside) {  // rare: the reference's walk around an unclamped query cell
        cnt = 0;
        w = 0.0f;
        const int64_t lx0 = cxu - 1 < 0 ? 0 : cxu - 1;
        const int64_t lx1 = cxu + 1 > (int64_t)g.nx - 1 ? (int64_t)g.nx - 1 : cxu + 1;
        for (int dz = -1; dz <= 1; dz++) {
            const int64_t nz = czu + dz;
            if (nz < 0 || nz >= (int64_t)g.nz) continue;
            for (int dy = -1; dy <= 1; dy++) {
                const int64_t ny = cyu + dy;
                if (ny < 0 || ny >= (int64_t)g.ny || lx0 > lx1) continue;
                const uint32_t row = (uint32_t)ny * g.nx + (uint32_t)nz * g.nx * g.ny;
                const uint32_t jb = cell_start[row + (uint32_t)lx0];
                const uint32_t je = min(cell_start[row + (uint32_t)lx1 + 1u], n);
                for (uint32_t j = jb; j < je; j++) nbr_pair(spos[j], q, radius_sq, coeff, cnt, w);
            }
        }
    }
    if (!in) return;
    const uint32_t i = sidx[s];
    if (i >= n) return;
    counts[i] = cnt;
    if (wsum) wsum[i] = w;
}

// Batched HashGrid::query_neighbors: one thread per query, neighbour positions read through
// sorted_indices from the caller's arrays exactly like hashgrid.rs:176-186.
__global__ __launch_bounds__(256) void k_query(const float* __restrict__ x,
                                               const float* __restrict__ y,
                                               const float* __restrict__ z, uint32_t stride,
                                               GridDesc g, const uint32_t* __restrict__ cstart,
                                               const uint32_t* __restrict__ sidx,
                                               const float* __restrict__ qx,
                                               const float* __restrict__ qy,
                                               const float* __restrict__ qz, uint32_t qstride,
                                               uint32_t nq, float radius_sq,
                                               uint32_t* __restrict__ counts,
                                               const uint32_t* __restrict__ offsets,
                                               uint32_t* __restrict__ indices) {
    uint32_t qi = blockIdx.x * blockDim.x + threadIdx.x;
    if (qi >= nq) return;
    size_t oq = (size_t)qi * qstride;
    const float px = qx[oq], py = qy[oq], pz = qz[oq];
    const int64_t cx = rust_as_i32(floorf((px - g.ox) / g.cs));
    const int64_t cy = rust_as_i32(floorf((py - g.oy) / g.cs));
    const int64_t cz = rust_as_i32(floorf((pz - g.oz) / g.cs));
    const int64_t x0 = cx - 1 < 0 ? 0 : cx - 1;
    const int64_t x1 = cx + 1 > (int64_t)g.nx - 1 ? (int64_t)g.nx - 1 : cx + 1;
    uint32_t cnt = 0;
    uint32_t* out = (offsets && indices) ? indices + offsets[qi] : nullptr;
    const uint32_t room = out ? offsets[qi + 1] - offsets[qi] : 0u;
    for (int dz = -1; dz <= 1; dz++) {
        int64_t nz = cz + dz;
        if (nz < 0 || nz >= (int64_t)g.nz) continue;
        for (int dy = -1; dy <= 1; dy++) {
            int64_t ny = cy + dy;
            if (ny < 0 || ny >= (int64_t)g.ny) continue;
            if (x0 > x1) continue;
            uint32_t row = (uint32_t)ny * g.nx + (uint32_t)nz * g.nx * g.ny;
            uint32_t b = cstart[row + (uint32_t)x0];
            uint32_t e = cstart[row + (uint32_t)x1 + 1u];
            for (uint32_t j = b; j < e; j++) {
                uint32_t pi = sidx[j];
                size_t o = (size_t)pi * stride;
                float dx = x[o] - px, dy2 = y[o] - py, dz2 = z[o] - pz;
                float dist_sq = dx * dx + dy2 * dy2 + dz2 * dz2;
                if (dist_sq <= radius_sq) {
                    if (cnt < room) out[cnt] = pi;
                    cnt++;
                }
            }
        }
    }
    counts[qi] = cnt;
}

hipError_t launch_query(fh_ctx* c, const float* x, const float* y, const float* z,
                        uint32_t stride, const GridDesc& g, const uint32_t* cell_start,
                        const uint32_t* sorted_indices, const float* qx, const float* qy,
                        const float* qz, uint32_t qstride, uint32_t nq, float radius,
                        uint32_t* counts, const uint32_t* offsets, uint32_t* indices) {
    if (nq == 0) return hipSuccess;
    k_query<<<ceil_div(nq, 256u), 256, 0, c->stream>>>(x, y, z, stride, g, cell_start,
                                                       sorted_indices, qx, qy, qz, qstride, nq,
                                                       radius * radius, counts, offsets, indices);
    return hipGetLastError();
}

hipError_t launch_neighbor_query(fh_ctx* c, const float* x, const float* y, const float* z,
                                 uint32_t stride, uint32_t n, const GridDesc& g,
                                 const uint32_t* cell_start, const uint32_t* sorted_indices,
                                 float radius, uint32_t* counts, float* wsum) {
    if (n == 0) return hipSuccess;
    // c->sout (3 float4 per point) is free between SPH calls: the packed copy goes there
    k_pack_pos<<<ceil_div(n, 256u), 256, 0, c->stream>>>(x, y, z, stride, n, c->sout);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_gather_pos<<<ceil_div(n, 256u), 256, 0, c->stream>>>(c->sout, sorted_indices, n, c->spos);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // Same float expressions as sph_density.rs:413-416 with h = radius.
    float h = radius;
    float h2 = h * h;
    float h9 = h2 * h2 * h2 * h2 * h;
    float coeff = 315.0f / (64.0f * 3.14159265f * h9);
    tbeg(c, KID_NBR);
    k_nbr_stream<<<ceil_div(n, (uint32_t)kWave), kWave, 0, c->stream>>>(
        c->spos, sorted_indices, n, g, cell_start, radius * radius, coeff, counts, wsum);
    tend(c, KID_NBR);
    return hipGetLastError();
}

}  // namespace fh
