// fh_sph.hip -- SPH density and fused pressure/viscosity passes for gfx950, plus the
// gravity / integrate / box modules.
//
// The passes run over the particles in cell-sorted order (gathered once per substep into
// float4 arrays), so a particle's 27-cell neighbourhood is 9 contiguous ranges of the same
// arrays -- the 3 x-adjacent cells of each (dy, dz) row -- and neighbour reads are coalesced
// and cache-friendly instead of the reference's gathers through sorted_idx into unsorted
// arrays (sph_density.rs:445-450).  Results are scattered back to the caller's arrays in
// original particle order, so FieldSet semantics are unchanged.
//
// Arithmetic follows the reference expressions term by term (the library is compiled with
// -ffp-contract=off and IEEE division / square root) and the neighbours of a particle are
// visited in the reference's order (dz, dy, dx, then ascending particle id within a cell), so
// density and velocity updates reproduce the CPU restatement of sph_density.rs:409-460 and
// sph_fused.rs:542-638.
#include "fh_internal.hpp"

namespace fh {

// Sorted-order copies of the state.  The sort's last pass wrote rank[i] = sorted slot of
// particle i; k_gather (particle order) writes spos[rank[i]] = (pos[i], bits of rank[i]) and
// svel[rank[i]] = (vel[i], bits of i) -- the caller's arrays are read in order and each
// particle costs two 16-byte stores, instead of six 4-byte reads from scattered lines.  The
// particle id in svel[.].w travels with the particle through later reorderings (co-located
// groups, resident substeps) and into the new state (k_finalize).
__global__ __launch_bounds__(256) void k_gather(
    const float* __restrict__ px, const float* __restrict__ py, const float* __restrict__ pz,
    const float* __restrict__ vx, const float* __restrict__ vy, const float* __restrict__ vz,
    const uint32_t* __restrict__ rank, uint32_t n, float4* __restrict__ spos,
    float4* __restrict__ svel) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t r = rank[i];
    if (r >= n) return;  // never taken when the sort is consistent
    spos[r] = make_float4(px[i], py[i], pz[i], __uint_as_float(r));
    if (svel) svel[r] = make_float4(vx[i], vy[i], vz[i], __uint_as_float(i));
}

// CSR cell ranges straight from the sorted keys, no scan: the key in slot s starts its run when
// the key before it, pk, differs; slot s then writes cell_start[c] = s for the cells
// pk < c <= k (the empty cells before its own take its index: the first sorted index with key
// >= c), and the last slot also writes n for the cells after its key up to and including C.
// These ranges partition 0..C, so every entry is written once; together they are the prefix
// sum of the per-cell counts of hashgrid.rs:102-106.  Short ranges are written by their lane,
// long ones by the whole wave.
__device__ __forceinline__ void fill_cells(uint32_t* __restrict__ cell_start, uint32_t lo,
                                           uint32_t hi, uint32_t val, int lane) {
    const bool mine = hi - lo <= 8u;
    if (mine)
        for (uint32_t c = lo; c < hi; c++) cell_start[c] = val;
    uint64_t wide = __ballot(!mine);
    while (wide) {  // uniform
        const int l = __ffsll((unsigned long long)wide) - 1;
        wide &= wide - 1ull;
        const uint32_t wlo = (uint32_t)__shfl((int)lo, l, kWave);
        const uint32_t whi = (uint32_t)__shfl((int)hi, l, kWave);
        const uint32_t wv = (uint32_t)__shfl((int)val, l, kWave);
        for (uint32_t c = wlo + (uint32_t)lane; c < whi; c += kWave) cell_start[c] = wv;
    }
}

// Cell ranges, and (big != null) the candidate co-located groups: runs of at least
// kCollapseMin keys in which at least kGroupHits of kGroupSamples evenly spaced particles (over
// the first L of the run, L its length rounded down to a power of two) sit at the position of
// one of them.  Listed as (first slot, offset of that sample) -- the group pass counts the run
// and the members at that sample's position exactly -- and tagged with the epoch in
// cand_tag[cell] for the plan, which runs beside the group pass.
template <class Pos>
__device__ __forceinline__ void cell_starts_slot(uint32_t s, const uint32_t* __restrict__ skeys,
                                                 uint32_t n, uint32_t C,
                                                 uint32_t* __restrict__ cell_start, Pos pos,
                                                 uint2* __restrict__ big, uint32_t cap,
                                                 uint64_t* __restrict__ cand_tag, Control* ctl) {
    const int lane = threadIdx.x & 63;
    uint32_t lo = 0, hi = 0, lo2 = 0, hi2 = 0;
    bool cand = false;
    uint32_t k = 0;
    if (s < n) {
        k = skeys[s];
        const uint32_t pk = s > 0u ? skeys[s - 1u] : 0xFFFFFFFFu;  // "-1" before slot 0
        if (pk != k) {
            lo = pk + 1u;
            hi = min(k, C - 1u) + 1u;
            cand = big && s + kCollapseMin - 1u < n && skeys[s + kCollapseMin - 1u] == k;
        }
        if (s == n - 1u) {
            lo2 = min(k, C - 1u) + 1u;
            hi2 = C + 1u;
        }
    }
    fill_cells(cell_start, lo, hi, s, lane);
    fill_cells(cell_start, lo2, hi2, n, lane);
    // Rare: a run of at least kCollapseMin.  The whole wave takes each such run of its lanes in
    // turn: lane q < kGroupSamples loads sample q (one round trip for all 16); the middle sample
    // is tried first as the group's position, then each other in turn (a corner group can fill
    // all but the middle of a run).
    uint64_t todo = __ballot(cand);
    while (todo) {  // uniform
        const int l = __ffsll((unsigned long long)todo) - 1;
        todo &= todo - 1ull;
        const uint32_t rs = (uint32_t)__builtin_amdgcn_readlane((int)s, l);
        const uint32_t rk = (uint32_t)__builtin_amdgcn_readlane((int)k, l);
        uint32_t L = kCollapseMin;
        while (L < (1u << 30) && rs + 2u * L - 1u < n && skeys[rs + 2u * L - 1u] == rk) L *= 2u;
        uint32_t px = 0, py = 0, pz = 0;
        if ((uint32_t)lane < kGroupSamples) {
            const float4 v = pos(rs + ((uint32_t)lane * L) / kGroupSamples);
            px = __float_as_uint(v.x);
            py = __float_as_uint(v.y);
            pz = __float_as_uint(v.z);
        }
        uint32_t off = 0, hits = 0;
        for (uint32_t a = 0; a < kGroupSamples; a++) {  // uniform
            const uint32_t qa = a == 0u ? kGroupSamples / 2u : (a <= kGroupSamples / 2u ? a - 1u : a);
            const uint32_t ax = (uint32_t)__builtin_amdgcn_readlane((int)px, (int)qa);
            const uint32_t ay = (uint32_t)__builtin_amdgcn_readlane((int)py, (int)qa);
            const uint32_t az = (uint32_t)__builtin_amdgcn_readlane((int)pz, (int)qa);
            const uint32_t hq = (uint32_t)__popcll(__ballot((uint32_t)lane < kGroupSamples &&
                                                            px == ax && py == ay && pz == az));
            if (hits < kGroupHits) {
                hits = hq;
                off = (qa * L) / kGroupSamples;
            }
        }
        if (hits >= kGroupHits && lane == 0) {
            const uint32_t slot = atomicAdd(&ctl->big_count.v, 1u);
            if (slot < cap) big[slot] = make_uint2(rs, off);
            cand_tag[rk] = (uint64_t)ctl->epoch << 32;  // the plan: this cell may hold a group
        }
    }
}

// Position of sorted slot x for the samples of cell_starts_slot: from the sorted copy, or, in
// resident substeps (which build that copy in the same kernel), from the previous substep's
// state through the slot map.
struct SortedPos {
    const float4* __restrict__ spos;
    __device__ float4 operator()(uint32_t x) const { return spos[x]; }
};
struct ResidentPos {
    const float4* __restrict__ sout;
    const uint32_t* __restrict__ prev;
    uint32_t n;
    __device__ float4 operator()(uint32_t x) const { return sout[2u * min(prev[x], n - 1u)]; }
};

__global__ __launch_bounds__(256) void k_cell_starts(const uint32_t* __restrict__ skeys,
                                                     uint32_t n, uint32_t C,
                                                     uint32_t* __restrict__ cell_start,
                                                     const float4* __restrict__ spos,
                                                     uint2* __restrict__ big, uint32_t cap,
                                                     uint64_t* __restrict__ cand_tag,
                                                     Control* ctl) {
    cell_starts_slot(blockIdx.x * blockDim.x + threadIdx.x, skeys, n, C, cell_start,
                     SortedPos{spos}, big, cap, cand_tag, ctl);
}

static hipError_t launch_cell_starts(fh_ctx* c, uint32_t cells, uint32_t n, bool list_big) {
    tbeg(c, KID_SCAN);
    k_cell_starts<<<ceil_div(n, 256u), 256, 0, c->stream>>>(
        c->skeys, n, cells, c->cell_start, c->spos, list_big ? c->big : nullptr,
        ceil_div(c->max_n, 64u) + 1u, c->run_tag, c->ctl);
    tend(c, KID_SCAN);
    return hipGetLastError();
}

hipError_t launch_gather(fh_ctx* c, const GridDesc& g, uint32_t cells, const float* px,
                         const float* py, const float* pz, const float* vx, const float* vy,
                         const float* vz, uint32_t n, bool with_vel, bool list_big) {
    (void)g;
    if (n == 0) return launch_fill_u32(c, c->cell_start, 0u, cells + 1u);
    tbeg(c, KID_GATHER);
    k_gather<<<ceil_div(n, 256u), 256, 0, c->stream>>>(px, py, pz, vx, vy, vz, c->rank, n,
                                                       c->spos, with_vel ? c->svel : nullptr);
    hipError_t e = hipGetLastError();
    tend(c, KID_GATHER);
    if (e != hipSuccess) return e;
    return launch_cell_starts(c, cells, n, list_big);
}

// Resident substeps: new slot r takes the state of previous slot prev[r] from c->sout (one
// 32-byte read: (x, y, z, rho), (vx, vy, vz, particle id)) and writes spos / svel in order;
// the same thread then does k_cell_starts' work for slot r.
__global__ __launch_bounds__(256) void k_gather_resident(
    const float4* __restrict__ sout, const uint32_t* __restrict__ prev, uint32_t n,
    float4* __restrict__ spos, float4* __restrict__ svel, const uint32_t* __restrict__ skeys,
    uint32_t C, uint32_t* __restrict__ cell_start, uint2* __restrict__ big, uint32_t cap,
    uint64_t* __restrict__ cand_tag, Control* ctl) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r < n) {
        const uint32_t q = prev[r];
        if (q < n) {  // always, when the sort is consistent
            const float4 p = sout[2u * q], v = sout[2u * q + 1u];
            spos[r] = make_float4(p.x, p.y, p.z, __uint_as_float(r));
            svel[r] = v;
        }
    }
    cell_starts_slot(r, skeys, n, C, cell_start, ResidentPos{sout, prev, n}, big, cap, cand_tag,
                     ctl);
}

hipError_t launch_gather_resident(fh_ctx* c, uint32_t cells, uint32_t n) {
    if (n == 0) return launch_fill_u32(c, c->cell_start, 0u, cells + 1u);
    tbeg(c, KID_GATHER);
    k_gather_resident<<<ceil_div(n, 256u), 256, 0, c->stream>>>(
        c->sout, c->sidx2, n, c->spos, c->svel, c->skeys, cells, c->cell_start, c->big,
        ceil_div(c->max_n, 64u) + 1u, c->run_tag, c->ctl);
    tend(c, KID_GATHER);
    return hipGetLastError();
}

// CSR cell_start from keys the caller already sorted (hashgrid.rs:102-106 computes the same
// array as the prefix sum of per-cell counts): cell_start[c] = number of keys < c for
// c = 0..C, so keys >= C count in no cell.  Each slot fills the cells between the previous
// slot's key and its own (both clamped to C), the last slot the cells after its key; the
// filled ranges partition 0..C.
__global__ __launch_bounds__(256) void k_csr_from_sorted(const uint32_t* __restrict__ keys,
                                                         uint32_t n, uint32_t C,
                                                         uint32_t* __restrict__ cell_start) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = threadIdx.x & 63;
    uint32_t lo = 0, hi = 0, lo2 = 0, hi2 = 0;
    if (s < n) {
        const uint32_t k = min(keys[s], C);
        const uint32_t lo_k = s > 0u ? min(keys[s - 1u], C) + 1u : 0u;  // "-1" before slot 0
        lo = lo_k;
        hi = lo_k <= k ? k + 1u : lo_k;
        if (s == n - 1u) {
            lo2 = k + 1u;
            hi2 = C + 1u;
        }
    }
    fill_cells(cell_start, lo, hi, s, lane);
    fill_cells(cell_start, lo2, hi2, n, lane);
}

hipError_t launch_csr_from_sorted(fh_ctx* c, const uint32_t* keys, uint32_t n, uint32_t cells,
                                  uint32_t* cell_start) {
    if (n == 0) return launch_fill_u32(c, cell_start, 0u, cells + 1u);
    k_csr_from_sorted<<<ceil_div(n, 256u), 256, 0, c->stream>>>(keys, n, cells, cell_start);
    return hipGetLastError();
}

// Sorted-order state for the exact force pass over a caller's grid (sorted_indices[s] = the
// particle in slot s): the same layout k_gather writes, plus the densities.
__global__ __launch_bounds__(256) void k_gather_grid(
    const float* __restrict__ px, const float* __restrict__ py, const float* __restrict__ pz,
    const float* __restrict__ vx, const float* __restrict__ vy, const float* __restrict__ vz,
    const float* __restrict__ density, const uint32_t* __restrict__ sorted_indices, uint32_t n,
    float4* __restrict__ spos, float4* __restrict__ svel, float* __restrict__ srho,
    uint32_t* __restrict__ sidx) {
    const uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const uint32_t i = sorted_indices[s];
    const bool ok = i < n;  // a malformed id reads particle 0 and is never written back
    const uint32_t q = ok ? i : 0u;
    spos[s] = make_float4(px[q], py[q], pz[q], __uint_as_float(s));
    svel[s] = make_float4(vx[q], vy[q], vz[q], __uint_as_float(q));
    srho[s] = density[q];
    sidx[s] = ok ? i : 0xFFFFFFFFu;
}

hipError_t launch_gather_grid(fh_ctx* c, const float* px, const float* py, const float* pz,
                              const float* vx, const float* vy, const float* vz,
                              const float* density, const uint32_t* sorted_indices, uint32_t n) {
    if (n == 0) return hipSuccess;
    tbeg(c, KID_GATHER);
    k_gather_grid<<<ceil_div(n, 256u), 256, 0, c->stream>>>(px, py, pz, vx, vy, vz, density,
                                                            sorted_indices, n, c->spos, c->svel,
                                                            c->srho, c->sidx);
    tend(c, KID_GATHER);
    return hipGetLastError();
}

// Binary position frame of the streaming runner (manifest_runner.rs:150-167 interleaves
// pos_x/y/z per particle; serve.rs:43-62 packs u32 frame, u32 count, then the f32 values,
// all little-endian -- the device's byte order).  Word w of the output is written by thread
// w (coalesced stores): words 0 and 1 are the header, word 2 + 3 i + a is component a of
// particle i.  The frame number is `frame`, or, when `counter` is non-NULL, *counter, which the
// kernel then increments (so a captured graph emits consecutive frame numbers).
__global__ __launch_bounds__(256) void k_pack_frame(const float* __restrict__ px,
                                                    const float* __restrict__ py,
                                                    const float* __restrict__ pz, uint32_t n,
                                                    uint32_t frame, uint32_t* counter,
                                                    uint32_t* __restrict__ out) {
    const uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t words = 2ull + 3ull * n;
    if (w >= words) return;
    if (w < 2u) {
        if (w == 0u) {
            uint32_t f = frame;
            if (counter) {
                f = *counter;
                *counter = f + 1u;  // one thread of one workgroup: no other access in the launch
            }
            out[0] = f;
        } else {
            out[1] = n;
        }
        return;
    }
    const uint64_t t = w - 2u;
    const uint32_t i = (uint32_t)(t / 3u), a = (uint32_t)(t - 3u * (t / 3u));
    const float* src = a == 0u ? px : (a == 1u ? py : pz);
    out[w] = __float_as_uint(src[i]);
}

hipError_t launch_pack_frame(fh_ctx* c, const float* px, const float* py, const float* pz,
                             uint32_t n, uint32_t frame, uint32_t* counter, void* out) {
    const uint64_t words = 2ull + 3ull * n;
    k_pack_frame<<<(uint32_t)((words + 255u) / 256u), 256, 0, c->stream>>>(
        px, py, pz, n, frame, counter, (uint32_t*)out);
    return hipGetLastError();
}

// Clamped cell of a particle in the SPH kernels (sph_density.rs:421-426): grid origin 0.
struct Cell3 {
    int cx, cy, cz;
};
__device__ __forceinline__ Cell3 sph_cell(const float4& p, const GridDesc& g) {
    Cell3 c;
    c.cx = (int)cell_coord(p.x, 0.0f, g.cs, g.nx);
    c.cy = (int)cell_coord(p.y, 0.0f, g.cs, g.ny);
    c.cz = (int)cell_coord(p.z, 0.0f, g.cs, g.nz);
    return c;
}

// ---------------------------------------------------------------------------------------------
// Density: rho_i = sum_j mass*poly6*(h2 - r2)^3 over r2 < h2, self included.
__global__ __launch_bounds__(256) void k_density(const float4* __restrict__ spos,
                                                 const uint32_t* __restrict__ sidx, uint32_t n,
                                                 GridDesc g, const uint32_t* __restrict__ cstart,
                                                 float h2, float mc, float* __restrict__ srho,
                                                 float* __restrict__ density) {
    uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const float4 pi = spos[s];
    const Cell3 c = sph_cell(pi, g);
    const int x0 = c.cx > 0 ? c.cx - 1 : 0;
    const int x1 = c.cx + 1 < (int)g.nx ? c.cx + 1 : (int)g.nx - 1;
    float rho = 0.0f;
    for (int dz = -1; dz <= 1; dz++) {
        int nz = c.cz + dz;
        if (nz < 0 || nz >= (int)g.nz) continue;
        for (int dy = -1; dy <= 1; dy++) {
            int ny = c.cy + dy;
            if (ny < 0 || ny >= (int)g.ny) continue;
            uint32_t row = (uint32_t)ny * g.nx + (uint32_t)nz * g.nx * g.ny;
            uint32_t b = cstart[row + (uint32_t)x0], e = min(cstart[row + (uint32_t)x1 + 1u], n);
            for (uint32_t j = b; j < e; j++) {
                float4 q = spos[j];
                float dx2 = pi.x - q.x;
                float dy2 = pi.y - q.y;
                float dz2 = pi.z - q.z;
                float r2 = dx2 * dx2 + dy2 * dy2 + dz2 * dz2;
                if (r2 < h2) {
                    float diff = h2 - r2;
                    rho += mc * diff * diff * diff;
                }
            }
        }
    }
    srho[s] = rho;
    const uint32_t i = sidx[s];
    if (density && i < n) density[i] = rho;
}

hipError_t launch_density(fh_ctx* c, const SphArgs& a, const uint32_t* cell_start,
                          float* density_out) {
    if (a.n == 0) return hipSuccess;
    // Same float expressions as sph_density.rs:413-416; mass * coeff is the first product of
    // `mass * poly6_coeff * diff * diff * diff` (:453).
    float h2 = a.h * a.h;
    float h9 = h2 * h2 * h2 * h2 * a.h;
    float poly6 = 315.0f / (64.0f * 3.14159265f * h9);
    float mc = a.mass * poly6;
    tbeg(c, KID_DENSITY);
    k_density<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->spos, c->sidx, a.n, a.g, cell_start,
                                                          h2, mc, c->srho, density_out);
    tend(c, KID_DENSITY);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
struct ForceConsts {
    float h, h2, mass, k, rho0, mu, gcoef, lcoef, dt;
    uint32_t flags;
    float gx, gy, gz;
    float mn[3], mx[3], e;
};

// Fused pressure + viscosity (sph_fused.rs:542-638) and the optional epilogue: gravity
// (gravity.rs:33), integrate with its non-finite guard (integrate.rs:23-29) and the box
// (box_collider.rs:37-46), written back through sidx to the caller's arrays.
__global__ __launch_bounds__(256) void k_force(const float4* __restrict__ spos,
                                               const float4* __restrict__ svel,
                                               const float* __restrict__ srho,
                                               const uint32_t* __restrict__ sidx, uint32_t n,
                                               GridDesc g, const uint32_t* __restrict__ cstart,
                                               ForceConsts K, float* __restrict__ px,
                                               float* __restrict__ py, float* __restrict__ pz,
                                               float* __restrict__ vx, float* __restrict__ vy,
                                               float* __restrict__ vz,
                                               float* __restrict__ accel) {
    uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= n) return;
    const float4 pi = spos[s];
    const float4 vi = svel[s];
    const float rho_i = srho[s];
    float ax = 0.0f, ay = 0.0f, az = 0.0f;
    float nvx = vi.x, nvy = vi.y, nvz = vi.z;
    if (!(rho_i < 1e-6f)) {
        const float p_i = K.k * (rho_i - K.rho0);
        float pax = 0.0f, pay = 0.0f, paz = 0.0f;
        float vax = 0.0f, vay = 0.0f, vaz = 0.0f;
        const Cell3 c = sph_cell(pi, g);
        const int x0 = c.cx > 0 ? c.cx - 1 : 0;
        const int x1 = c.cx + 1 < (int)g.nx ? c.cx + 1 : (int)g.nx - 1;
        for (int dz = -1; dz <= 1; dz++) {
            int nz = c.cz + dz;
            if (nz < 0 || nz >= (int)g.nz) continue;
            for (int dy = -1; dy <= 1; dy++) {
                int ny = c.cy + dy;
                if (ny < 0 || ny >= (int)g.ny) continue;
                uint32_t row = (uint32_t)ny * g.nx + (uint32_t)nz * g.nx * g.ny;
                uint32_t b = cstart[row + (uint32_t)x0], e = min(cstart[row + (uint32_t)x1 + 1u], n);
                for (uint32_t j = b; j < e; j++) {
                    float4 q = spos[j];
                    float djx = pi.x - q.x;
                    float djy = pi.y - q.y;
                    float djz = pi.z - q.z;
                    float r2 = djx * djx + djy * djy + djz * djz;
                    if (r2 < K.h2 && r2 > 1e-12f) {
                        float r = sqrtf(r2);
                        float rho_j = srho[j];
                        if (rho_j < 1e-6f) continue;
                        float diff = K.h - r;
                        float p_j = K.k * (rho_j - K.rho0);
                        float grad_scale = K.gcoef * diff * diff / r;
                        float f_scale = -K.mass * (p_i + p_j) / (2.0f * rho_j) * grad_scale;
                        pax += f_scale * djx;
                        pay += f_scale * djy;
                        paz += f_scale * djz;
                        float4 vj = svel[j];
                        float lap = K.lcoef * diff;
                        float v_scale = K.mu * K.mass / rho_j * lap;
                        vax += v_scale * (vj.x - vi.x);
                        vay += v_scale * (vj.y - vi.y);
                        vaz += v_scale * (vj.z - vi.z);
                    }
                }
            }
        }
        float inv_rho = 1.0f / rho_i;
        ax = (pax + vax) * inv_rho;
        ay = (pay + vay) * inv_rho;
        az = (paz + vaz) * inv_rho;
        nvx = vi.x + ax * K.dt;
        nvy = vi.y + ay * K.dt;
        nvz = vi.z + az * K.dt;
    }
    const uint32_t i = sidx[s];
    if (i >= n) return;
    float npx = pi.x, npy = pi.y, npz = pi.z;
    if (K.flags & FH_EPI_GRAVITY) {
        nvx += K.gx * K.dt;
        nvy += K.gy * K.dt;
        nvz += K.gz * K.dt;
    }
    if (K.flags & FH_EPI_INTEGRATE) {
        if (!isfinite(nvx)) nvx = 0.0f;
        if (!isfinite(nvy)) nvy = 0.0f;
        if (!isfinite(nvz)) nvz = 0.0f;
        npx += nvx * K.dt;
        npy += nvy * K.dt;
        npz += nvz * K.dt;
    }
    if (K.flags & FH_EPI_BOX) {
        if (npx < K.mn[0]) { npx = K.mn[0]; nvx = fabsf(nvx) * K.e; }
        if (npx > K.mx[0]) { npx = K.mx[0]; nvx = -fabsf(nvx) * K.e; }
        if (npy < K.mn[1]) { npy = K.mn[1]; nvy = fabsf(nvy) * K.e; }
        if (npy > K.mx[1]) { npy = K.mx[1]; nvy = -fabsf(nvy) * K.e; }
        if (npz < K.mn[2]) { npz = K.mn[2]; nvz = fabsf(nvz) * K.e; }
        if (npz > K.mx[2]) { npz = K.mx[2]; nvz = -fabsf(nvz) * K.e; }
    }
    vx[i] = nvx;
    vy[i] = nvy;
    vz[i] = nvz;
    if (K.flags & (FH_EPI_INTEGRATE | FH_EPI_BOX)) {
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

hipError_t launch_force(fh_ctx* c, const SphArgs& a, const fh_epilogue* epi,
                        const uint32_t* cell_start, float* px, float* py, float* pz, float* vx,
                        float* vy, float* vz, float* accel) {
    if (a.n == 0) return hipSuccess;
    ForceConsts K;
    K.h = a.h;
    K.h2 = a.h * a.h;
    K.mass = a.mass;
    K.k = a.k;
    K.rho0 = a.rho0;
    K.mu = a.mu;
    // sph_fused.rs:552-555
    float h6 = K.h2 * K.h2 * K.h2;
    K.gcoef = -45.0f / (3.14159265f * h6);
    K.lcoef = 45.0f / (3.14159265f * h6);
    K.dt = a.dt;
    K.flags = epi ? epi->flags : 0u;
    K.gx = epi ? epi->gravity[0] : 0.0f;
    K.gy = epi ? epi->gravity[1] : 0.0f;
    K.gz = epi ? epi->gravity[2] : 0.0f;
    for (int q = 0; q < 3; q++) {
        K.mn[q] = epi ? epi->box_min[q] : 0.0f;
        K.mx[q] = epi ? epi->box_max[q] : 0.0f;
    }
    K.e = epi ? epi->restitution : 0.0f;
    tbeg(c, KID_FORCE);
    k_force<<<ceil_div(a.n, 256u), 256, 0, c->stream>>>(c->spos, c->svel, c->srho, c->sidx, a.n,
                                                        a.g, cell_start, K, px, py, pz, vx, vy,
                                                        vz, accel);
    tend(c, KID_FORCE);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// Unfused modules (sph_pressure.rs:28-112, sph_viscosity.rs:27-106): one thread per particle i
// in original order, neighbours through the caller's grid (cell_start[C+1], sorted_indices[n]
// left in the FieldSet by the density module), visited cell by cell in the reference's order
// (dz, dy, dx, then the cell's range), j == i skipped.  The reference expressions are kept term
// by term (no contraction, IEEE division and square root), so each velocity equals the CPU
// restatement's bit for bit.  Ranges and ids are clamped to n so a malformed grid cannot read
// out of bounds.
struct UnfusedConsts {
    float h, h2, mass, k, rho0, mu, coef, dt;
    uint32_t n;
};

template <class Pair>
__device__ __forceinline__ void unfused_walk(const float* __restrict__ px,
                                             const float* __restrict__ py,
                                             const float* __restrict__ pz,
                                             const float* __restrict__ density,
                                             const uint32_t* __restrict__ cstart,
                                             const uint32_t* __restrict__ sidx, GridDesc g,
                                             const UnfusedConsts& K, uint32_t i, float xi,
                                             float yi, float zi, Pair&& pair) {
    const int cx = (int)cell_coord(xi, 0.0f, g.cs, g.nx);
    const int cy = (int)cell_coord(yi, 0.0f, g.cs, g.ny);
    const int cz = (int)cell_coord(zi, 0.0f, g.cs, g.nz);
    for (int dz = -1; dz <= 1; dz++) {
        const int nzz = cz + dz;
        if (nzz < 0 || nzz >= (int)g.nz) continue;
        for (int dy = -1; dy <= 1; dy++) {
            const int nyy = cy + dy;
            if (nyy < 0 || nyy >= (int)g.ny) continue;
            for (int dx = -1; dx <= 1; dx++) {
                const int nxx = cx + dx;
                if (nxx < 0 || nxx >= (int)g.nx) continue;
                const uint32_t cell = (uint32_t)nxx + (uint32_t)nyy * g.nx +
                                      (uint32_t)nzz * g.nx * g.ny;
                const uint32_t end = min(cstart[cell + 1u], K.n);
                for (uint32_t s = cstart[cell]; s < end; s++) {
                    const uint32_t j = sidx[s];
                    if (j == i || j >= K.n) continue;
                    float djx = xi - px[j];
                    float djy = yi - py[j];
                    float djz = zi - pz[j];
                    float r2 = djx * djx + djy * djy + djz * djz;
                    if (r2 < K.h2 && r2 > 1e-12f) {
                        float r = sqrtf(r2);
                        float rho_j = density[j];
                        if (rho_j < 1e-6f) continue;
                        pair(j, djx, djy, djz, r, rho_j);
                    }
                }
            }
        }
    }
}

// sph_pressure.rs:34-111; K.coef = -45 / (pi h^6).  Pressure terms read positions and
// densities only, so v_i is updated in place.
__global__ __launch_bounds__(256) void k_pressure(const float* __restrict__ px,
                                                  const float* __restrict__ py,
                                                  const float* __restrict__ pz,
                                                  float* __restrict__ vx, float* __restrict__ vy,
                                                  float* __restrict__ vz,
                                                  const float* __restrict__ density,
                                                  const uint32_t* __restrict__ cstart,
                                                  const uint32_t* __restrict__ sidx, GridDesc g,
                                                  UnfusedConsts K) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= K.n) return;
    const float rho_i = density[i];
    if (rho_i < 1e-6f) return;
    const float p_i = K.k * (rho_i - K.rho0);
    float ax = 0.0f, ay = 0.0f, az = 0.0f;
    unfused_walk(px, py, pz, density, cstart, sidx, g, K, i, px[i], py[i], pz[i],
                 [&](uint32_t, float djx, float djy, float djz, float r, float rho_j) {
                     float diff = K.h - r;
                     float p_j = K.k * (rho_j - K.rho0);
                     float grad_scale = K.coef * diff * diff / r;
                     float f_scale = -K.mass * (p_i + p_j) / (2.0f * rho_j) * grad_scale;
                     ax += f_scale * djx;
                     ay += f_scale * djy;
                     az += f_scale * djz;
                 });
    vx[i] += (ax / rho_i) * K.dt;
    vy[i] += (ay / rho_i) * K.dt;
    vz[i] += (az / rho_i) * K.dt;
}

// Velocities before the viscosity pass (particle order), read for every neighbour.
__global__ __launch_bounds__(256) void k_copy_vel(const float* __restrict__ vx,
                                                  const float* __restrict__ vy,
                                                  const float* __restrict__ vz, uint32_t n,
                                                  float4* __restrict__ v0) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) v0[i] = make_float4(vx[i], vy[i], vz[i], 0.0f);
}

// sph_viscosity.rs:34-105; K.coef = 45 / (pi h^6).
__global__ __launch_bounds__(256) void k_viscosity(const float* __restrict__ px,
                                                   const float* __restrict__ py,
                                                   const float* __restrict__ pz,
                                                   const float4* __restrict__ v0,
                                                   float* __restrict__ vx, float* __restrict__ vy,
                                                   float* __restrict__ vz,
                                                   const float* __restrict__ density,
                                                   const uint32_t* __restrict__ cstart,
                                                   const uint32_t* __restrict__ sidx, GridDesc g,
                                                   UnfusedConsts K) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= K.n) return;
    const float rho_i = density[i];
    if (rho_i < 1e-6f) return;
    const float4 vi = v0[i];
    float ax = 0.0f, ay = 0.0f, az = 0.0f;
    unfused_walk(px, py, pz, density, cstart, sidx, g, K, i, px[i], py[i], pz[i],
                 [&](uint32_t j, float, float, float, float r, float rho_j) {
                     float lap = K.coef * (K.h - r);
                     float scale = K.mu * K.mass / rho_j * lap;
                     const float4 vj = v0[j];
                     ax += scale * (vj.x - vi.x);
                     ay += scale * (vj.y - vi.y);
                     az += scale * (vj.z - vi.z);
                 });
    vx[i] = vi.x + (ax / rho_i) * K.dt;
    vy[i] = vi.y + (ay / rho_i) * K.dt;
    vz[i] = vi.z + (az / rho_i) * K.dt;
}

hipError_t launch_unfused(fh_ctx* c, bool viscosity, const SphArgs& a, const float* px,
                          const float* py, const float* pz, float* vx, float* vy, float* vz,
                          const float* density, const uint32_t* cell_start,
                          const uint32_t* sorted_indices) {
    if (a.n == 0) return hipSuccess;
    UnfusedConsts K;
    K.h = a.h;
    K.h2 = a.h * a.h;
    K.mass = a.mass;
    K.k = a.k;
    K.rho0 = a.rho0;
    K.mu = a.mu;
    const float h6 = K.h2 * K.h2 * K.h2;  // sph_pressure.rs:47-50, sph_viscosity.rs:47-49
    K.coef = viscosity ? 45.0f / (3.14159265f * h6) : -45.0f / (3.14159265f * h6);
    K.dt = a.dt;
    K.n = a.n;
    const uint32_t blocks = ceil_div(a.n, 256u);
    if (!viscosity) {
        k_pressure<<<blocks, 256, 0, c->stream>>>(px, py, pz, vx, vy, vz, density, cell_start,
                                                  sorted_indices, a.g, K);
        return hipGetLastError();
    }
    k_copy_vel<<<blocks, 256, 0, c->stream>>>(vx, vy, vz, a.n, c->svel);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_viscosity<<<blocks, 256, 0, c->stream>>>(px, py, pz, c->svel, vx, vy, vz, density,
                                               cell_start, sorted_indices, a.g, K);
    return hipGetLastError();
}

// Copy of the grid of the last rebuild (CSR cell_start[C+1], sorted ids) into caller arrays:
// the FieldSet's u32 fields that the unfused modules read (sph_density.rs:44-74 keeps them).
__global__ __launch_bounds__(256) void k_copy_grid(const uint32_t* __restrict__ cs_in,
                                                   uint32_t cells1,
                                                   const uint32_t* __restrict__ si_in, uint32_t n,
                                                   uint32_t* __restrict__ cs_out,
                                                   uint32_t* __restrict__ si_out) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < cells1; t += stride)
        if (cs_out) cs_out[t] = cs_in[t];
    for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < n; t += stride)
        if (si_out) si_out[t] = si_in[t];
}

hipError_t launch_copy_grid(fh_ctx* c, uint32_t cells, uint32_t n, uint32_t* cell_start,
                            uint32_t* sorted_indices) {
    if (!cell_start && !sorted_indices) return hipSuccess;
    uint32_t blocks = ceil_div(max(cells + 1u, n), 256u);
    if (blocks > 2048u) blocks = 2048u;
    k_copy_grid<<<blocks, 256, 0, c->stream>>>(c->cell_start, cells + 1u, c->sidx, n, cell_start,
                                               sorted_indices);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// gravity.rs:31-34
__global__ void k_gravity(float* __restrict__ vx, float* __restrict__ vy, float* __restrict__ vz,
                          float gx, float gy, float gz, float dt, uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        vx[i] += gx * dt;
        vy[i] += gy * dt;
        vz[i] += gz * dt;
    }
}

// integrate.rs:16-31
__global__ void k_integrate(float* __restrict__ px, float* __restrict__ py,
                            float* __restrict__ pz, float* __restrict__ vx,
                            float* __restrict__ vy, float* __restrict__ vz, float dt,
                            uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float _vx = vx[i], _vy = vy[i], _vz = vz[i];
    if (!isfinite(_vx)) { _vx = 0.0f; vx[i] = 0.0f; }
    if (!isfinite(_vy)) { _vy = 0.0f; vy[i] = 0.0f; }
    if (!isfinite(_vz)) { _vz = 0.0f; vz[i] = 0.0f; }
    px[i] += _vx * dt;
    py[i] += _vy * dt;
    pz[i] += _vz * dt;
}

// box_collider.rs:26-47
__global__ void k_box(float* __restrict__ px, float* __restrict__ py, float* __restrict__ pz,
                      float* __restrict__ vx, float* __restrict__ vy, float* __restrict__ vz,
                      float mnx, float mny, float mnz, float mxx, float mxy, float mxz, float e,
                      uint32_t n) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float x = px[i], y = py[i], z = pz[i], u = vx[i], v = vy[i], w = vz[i];
    if (x < mnx) { x = mnx; u = fabsf(u) * e; }
    if (x > mxx) { x = mxx; u = -fabsf(u) * e; }
    if (y < mny) { y = mny; v = fabsf(v) * e; }
    if (y > mxy) { y = mxy; v = -fabsf(v) * e; }
    if (z < mnz) { z = mnz; w = fabsf(w) * e; }
    if (z > mxz) { z = mxz; w = -fabsf(w) * e; }
    px[i] = x;
    py[i] = y;
    pz[i] = z;
    vx[i] = u;
    vy[i] = v;
    vz[i] = w;
}

hipError_t launch_gravity(fh_ctx* c, float* vx, float* vy, float* vz, uint32_t n, float gx,
                          float gy, float gz, float dt) {
    if (n == 0) return hipSuccess;
    k_gravity<<<ceil_div(n, 256u), 256, 0, c->stream>>>(vx, vy, vz, gx, gy, gz, dt, n);
    return hipGetLastError();
}

hipError_t launch_integrate(fh_ctx* c, float* px, float* py, float* pz, float* vx, float* vy,
                            float* vz, uint32_t n, float dt) {
    if (n == 0) return hipSuccess;
    k_integrate<<<ceil_div(n, 256u), 256, 0, c->stream>>>(px, py, pz, vx, vy, vz, dt, n);
    return hipGetLastError();
}

hipError_t launch_box(fh_ctx* c, float* px, float* py, float* pz, float* vx, float* vy,
                      float* vz, uint32_t n, const float* mn, const float* mx, float e) {
    if (n == 0) return hipSuccess;
    k_box<<<ceil_div(n, 256u), 256, 0, c->stream>>>(px, py, pz, vx, vy, vz, mn[0], mn[1], mn[2],
                                                    mx[0], mx[1], mx[2], e, n);
    return hipGetLastError();
}

}  // namespace fh
