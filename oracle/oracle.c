/*
 * oracle.c -- CPU restatement of forge-gpu's SPH / hash-grid path (TEST INFRASTRUCTURE ONLY).
 *
 * The checker for the HIP path.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  Built with -O2 -ffp-contract=off: every float expression below
 * is evaluated as written, left to right, without FMA, like the reference's Rust CPU code.
 * Citations are reference file:line (paths relative to the huaying/forge-gpu repository root).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Rust `f32 as i32` (saturating cast, NaN -> 0).  hashgrid.rs:129-131 applies it to floor(). */
int32_t or_f32_as_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return INT32_MAX;
    if (f <= -2147483648.0f) return INT32_MIN;
    return (int32_t)f;
}

/* hashgrid.rs:128-139 */
uint32_t or_position_to_cell(float x, float y, float z, float cell_size, const float origin[3],
                             const uint32_t dims[3]) {
    int32_t cx = or_f32_as_i32(floorf((x - origin[0]) / cell_size));
    int32_t cy = or_f32_as_i32(floorf((y - origin[1]) / cell_size));
    int32_t cz = or_f32_as_i32(floorf((z - origin[2]) / cell_size));
    /* cx.max(0).min(dim as i32 - 1) as u32 */
    int32_t mx = (int32_t)dims[0] - 1, my = (int32_t)dims[1] - 1, mz = (int32_t)dims[2] - 1;
    if (cx < 0) cx = 0;
    if (cx > mx) cx = mx;
    if (cy < 0) cy = 0;
    if (cy > my) cy = my;
    if (cz < 0) cz = 0;
    if (cz > mz) cz = mz;
    /* cx + cy * dim_x + cz * dim_x * dim_y in u32 (wrapping) */
    return (uint32_t)cx + (uint32_t)cy * dims[0] + (uint32_t)cz * dims[0] * dims[1];
}

/* hashgrid.rs:89-92 */
void or_hash_cells(const float* x, const float* y, const float* z, uint32_t stride, uint32_t n,
                   float cell_size, const float origin[3], const uint32_t dims[3],
                   uint32_t* keys, uint32_t* vals) {
    for (uint32_t i = 0; i < n; i++) {
        size_t o = (size_t)i * stride;
        keys[i] = or_position_to_cell(x[o], y[o], z[o], cell_size, origin, dims);
        if (vals) vals[i] = i;
    }
}

/* Stable sort by masked key (tests/radix_sort_test.rs:111-113 `sort_by_key` order).  Bottom-up
 * merge sort: on equal masked keys the left run wins, so input order is kept. */
int or_stable_sort_pairs(uint32_t* keys, uint32_t* vals, uint32_t n, uint32_t num_bits) {
    if (num_bits < 1 || num_bits > 32) return -1;
    if (n < 2) return 0;
    uint32_t mask = num_bits == 32 ? 0xFFFFFFFFu : ((1u << num_bits) - 1u);
    uint32_t* tk = (uint32_t*)malloc((size_t)n * 4);
    uint32_t* tv = (uint32_t*)malloc((size_t)n * 4);
    if (!tk || !tv) {
        free(tk);
        free(tv);
        return -1;
    }
    uint32_t *sk = keys, *sv = vals, *dk = tk, *dv = tv;
    for (size_t width = 1; width < n; width *= 2) {
        for (size_t lo = 0; lo < n; lo += 2 * width) {
            size_t mid = lo + width < n ? lo + width : n;
            size_t hi = lo + 2 * width < n ? lo + 2 * width : n;
            size_t a = lo, b = mid, o = lo;
            while (a < mid && b < hi) {
                if ((sk[b] & mask) < (sk[a] & mask)) {
                    dk[o] = sk[b];
                    dv[o++] = sv[b++];
                } else {
                    dk[o] = sk[a];
                    dv[o++] = sv[a++];
                }
            }
            while (a < mid) {
                dk[o] = sk[a];
                dv[o++] = sv[a++];
            }
            while (b < hi) {
                dk[o] = sk[b];
                dv[o++] = sv[b++];
            }
        }
        uint32_t* t = sk;
        sk = dk;
        dk = t;
        t = sv;
        sv = dv;
        dv = t;
    }
    if (sk != keys) {
        memcpy(keys, sk, (size_t)n * 4);
        memcpy(vals, sv, (size_t)n * 4);
    }
    free(tk);
    free(tv);
    return 0;
}

/* radix_sort.rs:259-293 (sentinel fill) and :451-465 (boundary kernel, one i at a time). */
void or_find_cell_boundaries(const uint32_t* sorted_keys, uint32_t n, uint32_t num_cells,
                             uint32_t* cell_start, uint32_t* cell_end) {
    for (uint32_t c = 0; c < num_cells; c++) {
        cell_start[c] = 0xFFFFFFFFu;
        cell_end[c] = 0;
    }
    for (uint32_t i = 0; i < n; i++) {
        uint32_t cell = sorted_keys[i];
        if (cell >= num_cells) continue; /* the reference kernel would write out of bounds */
        if (i == 0 || sorted_keys[i - 1] != cell) cell_start[cell] = i;
        if (i == n - 1 || sorted_keys[i + 1] != cell) cell_end[cell] = i + 1;
    }
}

/* hashgrid.rs:95-106 on already-sorted keys: counts, then starts[c+1] = starts[c] + counts[c]. */
void or_cell_start_csr(const uint32_t* sorted_keys, uint32_t n, uint32_t num_cells,
                       uint32_t* cell_start) {
    memset(cell_start, 0, ((size_t)num_cells + 1) * 4);
    for (uint32_t i = 0; i < n; i++)
        if (sorted_keys[i] < num_cells) cell_start[sorted_keys[i] + 1] += 1;
    for (uint32_t c = 0; c < num_cells; c++) cell_start[c + 1] += cell_start[c];
}

/* hashgrid.rs:82-125 */
int or_hashgrid_build(const float* x, const float* y, const float* z, uint32_t stride,
                      uint32_t n, float cell_size, const float origin[3], const uint32_t dims[3],
                      uint32_t* cell_start, uint32_t* sorted_indices, uint32_t* cell_indices) {
    uint32_t num_cells = dims[0] * dims[1] * dims[2];
    /* Step 1 (:89-92) */
    or_hash_cells(x, y, z, stride, n, cell_size, origin, dims, cell_indices, NULL);
    /* Step 2 (:95-100) */
    uint32_t* counts = (uint32_t*)calloc((size_t)num_cells + 1, 4);
    if (!counts) return -1;
    for (uint32_t i = 0; i < n; i++)
        if (cell_indices[i] < num_cells) counts[cell_indices[i]] += 1;
    /* Step 3 (:103-106) */
    cell_start[0] = 0;
    for (uint32_t c = 0; c < num_cells; c++) cell_start[c + 1] = cell_start[c] + counts[c];
    /* Step 4 (:109-117): stable scatter in ascending particle index */
    memcpy(counts, cell_start, (size_t)num_cells * 4);
    for (uint32_t i = 0; i < n; i++) {
        uint32_t c = cell_indices[i];
        if (c < num_cells) sorted_indices[counts[c]++] = i;
    }
    free(counts);
    return 0;
}

/* hashgrid.rs:145-193.  Query cell is not clamped (:155-157); out-of-range cells are skipped
 * (:169-170); diff = p_j - q and dist_sq = (dx*dx + dy*dy) + dz*dz <= r*r (:178-184). */
uint32_t or_query_neighbors(float qx, float qy, float qz, float radius, const float* x,
                            const float* y, const float* z, uint32_t stride, float cell_size,
                            const float origin[3], const uint32_t dims[3],
                            const uint32_t* cell_start, const uint32_t* sorted_indices,
                            uint32_t* out, uint32_t cap) {
    uint32_t found = 0;
    float radius_sq = radius * radius;
    int64_t cx = or_f32_as_i32(floorf((qx - origin[0]) / cell_size));
    int64_t cy = or_f32_as_i32(floorf((qy - origin[1]) / cell_size));
    int64_t cz = or_f32_as_i32(floorf((qz - origin[2]) / cell_size));
    for (int dz = -1; dz <= 1; dz++)
        for (int dy = -1; dy <= 1; dy++)
            for (int dx = -1; dx <= 1; dx++) {
                int64_t nx = cx + dx, ny = cy + dy, nz = cz + dz;
                if (nx < 0 || ny < 0 || nz < 0) continue;
                if (nx >= dims[0] || ny >= dims[1] || nz >= dims[2]) continue;
                uint32_t cell = (uint32_t)nx + (uint32_t)ny * dims[0] +
                                (uint32_t)nz * dims[0] * dims[1];
                for (uint32_t si = cell_start[cell]; si < cell_start[cell + 1]; si++) {
                    uint32_t pi = sorted_indices[si];
                    size_t o = (size_t)pi * stride;
                    float ddx = x[o] - qx, ddy = y[o] - qy, ddz = z[o] - qz;
                    float dist_sq = ddx * ddx + ddy * ddy + ddz * ddz;
                    if (dist_sq <= radius_sq) {
                        if (found < cap) out[found] = pi;
                        found++;
                    }
                }
            }
    return found;
}

/* Same walk as or_query_neighbors with q = p_i; weight as sph_density.rs:413-416/:452-453 with
 * h = radius and no mass factor: c * diff * diff * diff, diff = r^2 - dist_sq. */
void or_neighbor_counts(const float* x, const float* y, const float* z, uint32_t stride,
                        uint32_t n, float cell_size, const float origin[3],
                        const uint32_t dims[3], const uint32_t* cell_start,
                        const uint32_t* sorted_indices, float radius, uint32_t* counts,
                        float* wsum) {
    float radius_sq = radius * radius;
    float h2 = radius * radius;
    float h9 = h2 * h2 * h2 * h2 * radius;
    float coeff = 315.0f / (64.0f * 3.14159265f * h9);
    for (uint32_t i = 0; i < n; i++) {
        size_t oi = (size_t)i * stride;
        float qx = x[oi], qy = y[oi], qz = z[oi];
        int64_t cx = or_f32_as_i32(floorf((qx - origin[0]) / cell_size));
        int64_t cy = or_f32_as_i32(floorf((qy - origin[1]) / cell_size));
        int64_t cz = or_f32_as_i32(floorf((qz - origin[2]) / cell_size));
        uint32_t cnt = 0;
        float w = 0.0f;
        for (int dz = -1; dz <= 1; dz++)
            for (int dy = -1; dy <= 1; dy++)
                for (int dx = -1; dx <= 1; dx++) {
                    int64_t nx = cx + dx, ny = cy + dy, nz = cz + dz;
                    if (nx < 0 || ny < 0 || nz < 0) continue;
                    if (nx >= dims[0] || ny >= dims[1] || nz >= dims[2]) continue;
                    uint32_t cell = (uint32_t)nx + (uint32_t)ny * dims[0] +
                                    (uint32_t)nz * dims[0] * dims[1];
                    for (uint32_t si = cell_start[cell]; si < cell_start[cell + 1]; si++) {
                        size_t o = (size_t)sorted_indices[si] * stride;
                        float ddx = x[o] - qx, ddy = y[o] - qy, ddz = z[o] - qz;
                        float dist_sq = ddx * ddx + ddy * ddy + ddz * ddz;
                        if (dist_sq <= radius_sq) {
                            float diff = h2 - dist_sq;
                            cnt++;
                            w += coeff * diff * diff * diff;
                        }
                    }
                }
        counts[i] = cnt;
        if (wsum) wsum[i] = w;
    }
}

/* Clamped cell coordinate of the SPH kernels, sph_density.rs:421-426 / sph_fused.rs:91-96:
 * (int)floorf(p / cell_size) (PTX cvt.rzi saturates and maps NaN to 0, like Rust `as`). */
static int32_t sph_cell_coord(float p, float cell_size, uint32_t dim) {
    int32_t c = or_f32_as_i32(floorf(p / cell_size));
    if (c < 0) c = 0;
    if (c >= (int32_t)dim) c = (int32_t)dim - 1;
    return c;
}

/* sph_density.rs:409-460 */
/* Density of particle i, the body of the per-particle loop of sph_density.rs:401-461. */
static float density_one(const or_sph_params* p, const float* px, const float* py,
                         const float* pz, const uint32_t* cell_start,
                         const uint32_t* sorted_indices, uint32_t i) {
    const float h = p->h, mass = p->mass, cs = p->cell_size;
    const int32_t gnx = (int32_t)p->dims[0], gny = (int32_t)p->dims[1], gnz = (int32_t)p->dims[2];
    float h2 = h * h;
    float h9 = h2 * h2 * h2 * h2 * h;
    float poly6_coeff = 315.0f / (64.0f * 3.14159265f * h9);
    float xi = px[i], yi = py[i], zi = pz[i];
    float rho = 0.0f;
    int32_t cx = sph_cell_coord(xi, cs, p->dims[0]);
    int32_t cy = sph_cell_coord(yi, cs, p->dims[1]);
    int32_t cz = sph_cell_coord(zi, cs, p->dims[2]);
    for (int dz = -1; dz <= 1; dz++) {
        int32_t nz = cz + dz;
        if (nz < 0 || nz >= gnz) continue;
        for (int dy = -1; dy <= 1; dy++) {
            int32_t ny = cy + dy;
            if (ny < 0 || ny >= gny) continue;
            for (int dx = -1; dx <= 1; dx++) {
                int32_t nx = cx + dx;
                if (nx < 0 || nx >= gnx) continue;
                uint32_t cell = (uint32_t)nx + (uint32_t)ny * (uint32_t)gnx +
                                (uint32_t)nz * (uint32_t)gnx * (uint32_t)gny;
                uint32_t start = cell_start[cell], end = cell_start[cell + 1];
                for (uint32_t s = start; s < end; s++) {
                    uint32_t j = sorted_indices[s];
                    float dx2 = xi - px[j];
                    float dy2 = yi - py[j];
                    float dz2 = zi - pz[j];
                    float r2 = dx2 * dx2 + dy2 * dy2 + dz2 * dz2;
                    if (r2 < h2) {
                        float diff = h2 - r2;
                        rho += mass * poly6_coeff * diff * diff * diff;
                    }
                }
            }
        }
    }
    return rho;
}

void or_sph_density(const or_sph_params* p, const float* px, const float* py, const float* pz,
                    uint32_t n, const uint32_t* cell_start, const uint32_t* sorted_indices,
                    float* density) {
    for (uint32_t i = 0; i < n; i++)
        density[i] = density_one(p, px, py, pz, cell_start, sorted_indices, i);
}

void or_sph_density_at(const or_sph_params* p, const float* px, const float* py,
                       const float* pz, const uint32_t* cell_start,
                       const uint32_t* sorted_indices, const uint32_t* which, uint32_t m,
                       float* density) {
    for (uint32_t k = 0; k < m; k++)
        density[k] = density_one(p, px, py, pz, cell_start, sorted_indices, which[k]);
}

/* Per-pair maths of sph_fused.rs:542-638 (identical to sph_pressure.rs / sph_viscosity.rs
 * terms), neighbour set = the 27 clamped cells, velocities of neighbours from the input. */
void or_sph_force(const or_sph_params* p, const float* px, const float* py, const float* pz,
                  const float* vx, const float* vy, const float* vz, const float* density,
                  uint32_t n, const uint32_t* cell_start, const uint32_t* sorted_indices,
                  float dt, float* vout, float* accel) {
    const float h = p->h, mass = p->mass, cs = p->cell_size;
    const float gas_constant = p->gas_constant, rest_density = p->rest_density;
    const float visc_coeff = p->visc;
    const int32_t gnx = (int32_t)p->dims[0], gny = (int32_t)p->dims[1], gnz = (int32_t)p->dims[2];
    float h2 = h * h;
    float h6 = h2 * h2 * h2;
    float spiky_grad_coeff = -45.0f / (3.14159265f * h6);
    float visc_lap_coeff = 45.0f / (3.14159265f * h6);
    for (uint32_t i = 0; i < n; i++) {
        float xi = px[i], yi = py[i], zi = pz[i];
        float vxi = vx[i], vyi = vy[i], vzi = vz[i];
        float rho_i = density[i];
        float ax = 0.0f, ay = 0.0f, az = 0.0f;
        if (!(rho_i < 1e-6f)) { /* :550 -- particles with rho_i < 1e-6 are left untouched */
            float p_i = gas_constant * (rho_i - rest_density);
            float pax = 0.0f, pay = 0.0f, paz = 0.0f;
            float vax = 0.0f, vay = 0.0f, vaz = 0.0f;
            int32_t cx = sph_cell_coord(xi, cs, p->dims[0]);
            int32_t cy = sph_cell_coord(yi, cs, p->dims[1]);
            int32_t cz = sph_cell_coord(zi, cs, p->dims[2]);
            for (int dz = -1; dz <= 1; dz++)
                for (int dy = -1; dy <= 1; dy++)
                    for (int dx = -1; dx <= 1; dx++) {
                        int32_t ncx = cx + dx, ncy = cy + dy, ncz = cz + dz;
                        if (ncx < 0 || ncx >= gnx || ncy < 0 || ncy >= gny || ncz < 0 ||
                            ncz >= gnz)
                            continue;
                        uint32_t cell = (uint32_t)ncx + (uint32_t)ncy * (uint32_t)gnx +
                                        (uint32_t)ncz * (uint32_t)gnx * (uint32_t)gny;
                        for (uint32_t s = cell_start[cell]; s < cell_start[cell + 1]; s++) {
                            uint32_t j = sorted_indices[s];
                            float djx = xi - px[j];
                            float djy = yi - py[j];
                            float djz = zi - pz[j];
                            float r2 = djx * djx + djy * djy + djz * djz;
                            if (r2 < h2 && r2 > 1e-12f) {
                                float r = sqrtf(r2);
                                float rho_j = density[j];
                                if (rho_j < 1e-6f) continue;
                                float diff = h - r;
                                float p_j = gas_constant * (rho_j - rest_density);
                                float grad_scale = spiky_grad_coeff * diff * diff / r;
                                float f_scale = -mass * (p_i + p_j) / (2.0f * rho_j) * grad_scale;
                                pax += f_scale * djx;
                                pay += f_scale * djy;
                                paz += f_scale * djz;
                                float lap = visc_lap_coeff * diff;
                                float v_scale = visc_coeff * mass / rho_j * lap;
                                vax += v_scale * (vx[j] - vxi);
                                vay += v_scale * (vy[j] - vyi);
                                vaz += v_scale * (vz[j] - vzi);
                            }
                        }
                    }
            float inv_rho = 1.0f / rho_i;
            ax = (pax + vax) * inv_rho;
            ay = (pay + vay) * inv_rho;
            az = (paz + vaz) * inv_rho;
            if (vout) { /* :635-637 */
                vout[i] = vxi + ax * dt;
                vout[n + i] = vyi + ay * dt;
                vout[2 * (size_t)n + i] = vzi + az * dt;
            }
        } else if (vout) {
            vout[i] = vxi;
            vout[n + i] = vyi;
            vout[2 * (size_t)n + i] = vzi;
        }
        if (accel) {
            accel[i] = ax;
            accel[n + i] = ay;
            accel[2 * (size_t)n + i] = az;
        }
    }
}

/* Relative size of a pair distance's float32 rounding in the sensitivity scale: r^2 from
 * rounded differences, squares and sums (about 4 units of roundoff), then a square root or a
 * reciprocal square root (1-2 more), with a margin: 8 units of 2^-24. */
#define OR_DR_REL (8.0 / 16777216.0)

/* fp64 acceleration, error scale and distance-rounding sensitivity of particle i (body of
 * or_sph_force_f64's loop).  s = sum over pairs of |pressure term| + |viscosity term|;
 * e = sum over pairs of |d term / d r| * OR_DR_REL * r: (h - r) cancels for r near h, so a
 * float32 rounding of r changes such a term by far more than its own relative rounding. */
static void force64_one(const or_sph_params* p, const float* px, const float* py,
                        const float* pz, const float* vx, const float* vy, const float* vz,
                        const float* density, const uint32_t* cell_start,
                        const uint32_t* sorted_indices, uint32_t i, double a[3], double s[3],
                        double e[3]) {
    const double h = p->h, mass = p->mass;
    const double k = p->gas_constant, rho0 = p->rest_density, mu = p->visc;
    const int32_t gnx = (int32_t)p->dims[0], gny = (int32_t)p->dims[1], gnz = (int32_t)p->dims[2];
    const float h2f = p->h * p->h;
    const double PI = 3.14159265358979323846;
    double h6 = h * h * h * h * h * h;
    double gcoef = -45.0 / (PI * h6), lcoef = 45.0 / (PI * h6);
    for (int c = 0; c < 3; c++) a[c] = s[c] = e[c] = 0.0;
    float rho_if = density[i];
    if (rho_if < 1e-6f) return;
    double rho_i = rho_if, p_i = k * (rho_i - rho0);
    int32_t cx = sph_cell_coord(px[i], p->cell_size, p->dims[0]);
    int32_t cy = sph_cell_coord(py[i], p->cell_size, p->dims[1]);
    int32_t cz = sph_cell_coord(pz[i], p->cell_size, p->dims[2]);
    for (int dz = -1; dz <= 1; dz++)
        for (int dy = -1; dy <= 1; dy++)
            for (int dx = -1; dx <= 1; dx++) {
                int32_t ncx = cx + dx, ncy = cy + dy, ncz = cz + dz;
                if (ncx < 0 || ncx >= gnx || ncy < 0 || ncy >= gny || ncz < 0 || ncz >= gnz)
                    continue;
                uint32_t cell = (uint32_t)ncx + (uint32_t)ncy * (uint32_t)gnx +
                                (uint32_t)ncz * (uint32_t)gnx * (uint32_t)gny;
                for (uint32_t q = cell_start[cell]; q < cell_start[cell + 1]; q++) {
                    uint32_t j = sorted_indices[q];
                    float fx = px[i] - px[j], fy = py[i] - py[j], fz = pz[i] - pz[j];
                    float r2f = fx * fx + fy * fy + fz * fz;
                    if (!(r2f < h2f && r2f > 1e-12f)) continue;
                    if (density[j] < 1e-6f) continue;
                    double d[3] = {(double)px[i] - px[j], (double)py[i] - py[j],
                                   (double)pz[i] - pz[j]};
                    double r = sqrt(d[0] * d[0] + d[1] * d[1] + d[2] * d[2]);
                    double rho_j = density[j], p_j = k * (rho_j - rho0);
                    double diff = h - r;
                    double fsc = -mass * (p_i + p_j) / (2.0 * rho_j) * (gcoef * diff * diff / r);
                    double vsc = mu * mass / rho_j * (lcoef * diff);
                    double dv[3] = {(double)vx[j] - vx[i], (double)vy[j] - vy[i],
                                    (double)vz[j] - vz[i]};
                    /* d/dr of the pair factors (the direction d / r is well conditioned) */
                    double dfsc = -mass * (p_i + p_j) / (2.0 * rho_j) * (gcoef * 2.0 * diff / r);
                    double dvsc = mu * mass / rho_j * lcoef;
                    double dr = OR_DR_REL * r;
                    for (int c = 0; c < 3; c++) {
                        double tp = fsc * d[c], tv = vsc * dv[c];
                        a[c] += tp + tv;
                        s[c] += fabs(tp) + fabs(tv);
                        e[c] += (fabs(dfsc * d[c]) + fabs(dvsc * dv[c])) * dr;
                    }
                }
            }
    for (int c = 0; c < 3; c++) {
        a[c] /= rho_i;
        s[c] /= rho_i;
        e[c] /= rho_i;
    }
}

void or_sph_force_f64(const or_sph_params* p, const float* px, const float* py,
                      const float* pz, const float* vx, const float* vy, const float* vz,
                      const float* density, uint32_t n, const uint32_t* cell_start,
                      const uint32_t* sorted_indices, double* accel64, double* scale64,
                      double* sens64) {
    for (uint32_t i = 0; i < n; i++) {
        double a[3], s[3], e[3];
        force64_one(p, px, py, pz, vx, vy, vz, density, cell_start, sorted_indices, i, a, s, e);
        for (int c = 0; c < 3; c++) {
            accel64[(size_t)c * n + i] = a[c];
            scale64[(size_t)c * n + i] = s[c];
            if (sens64) sens64[(size_t)c * n + i] = e[c];
        }
    }
}

void or_sph_force_f64_at(const or_sph_params* p, const float* px, const float* py,
                         const float* pz, const float* vx, const float* vy, const float* vz,
                         const float* density, const uint32_t* cell_start,
                         const uint32_t* sorted_indices, const uint32_t* which, uint32_t m,
                         double* accel64, double* scale64, double* sens64) {
    for (uint32_t q = 0; q < m; q++) {
        double a[3], s[3], e[3];
        force64_one(p, px, py, pz, vx, vy, vz, density, cell_start, sorted_indices, which[q], a,
                    s, e);
        for (int c = 0; c < 3; c++) {
            accel64[(size_t)c * m + q] = a[c];
            scale64[(size_t)c * m + q] = s[c];
            if (sens64) sens64[(size_t)c * m + q] = e[c];
        }
    }
}

/* Shared walk of the unfused modules: calls the pair function for every j != i of the
 * 27-cell neighbourhood with r^2 < h^2 && r^2 > 1e-12 and rho_j >= 1e-6, in the reference's
 * order (dz, dy, dx, then the cell's range of sorted_indices), sph_pressure.rs:61-99 and
 * sph_viscosity.rs:58-97 (identical loops). */
typedef void (*or_pair_fn)(void* st, uint32_t j, float djx, float djy, float djz, float r,
                           float rho_j);

static void unfused_walk(const or_sph_params* p, const float* px, const float* py,
                         const float* pz, const float* density, const uint32_t* cell_start,
                         const uint32_t* sorted_indices, uint32_t i, or_pair_fn fn, void* st) {
    const float h = p->h, cs = p->cell_size;
    const int32_t gnx = (int32_t)p->dims[0], gny = (int32_t)p->dims[1], gnz = (int32_t)p->dims[2];
    float h2 = h * h;
    float xi = px[i], yi = py[i], zi = pz[i];
    int32_t cx = sph_cell_coord(xi, cs, p->dims[0]);
    int32_t cy = sph_cell_coord(yi, cs, p->dims[1]);
    int32_t cz = sph_cell_coord(zi, cs, p->dims[2]);
    for (int dz = -1; dz <= 1; dz++) {
        int32_t nzz = cz + dz;
        if (nzz < 0 || nzz >= gnz) continue;
        for (int dy = -1; dy <= 1; dy++) {
            int32_t nyy = cy + dy;
            if (nyy < 0 || nyy >= gny) continue;
            for (int dx = -1; dx <= 1; dx++) {
                int32_t nxx = cx + dx;
                if (nxx < 0 || nxx >= gnx) continue;
                uint32_t cell = (uint32_t)nxx + (uint32_t)nyy * (uint32_t)gnx +
                                (uint32_t)nzz * (uint32_t)gnx * (uint32_t)gny;
                uint32_t start = cell_start[cell];
                uint32_t end = cell_start[cell + 1];
                for (uint32_t s = start; s < end; s++) {
                    uint32_t j = sorted_indices[s];
                    if (j == i) continue;
                    float djx = xi - px[j];
                    float djy = yi - py[j];
                    float djz = zi - pz[j];
                    float r2 = djx * djx + djy * djy + djz * djz;
                    if (r2 < h2 && r2 > 1e-12f) {
                        float r = sqrtf(r2);
                        float rho_j = density[j];
                        if (rho_j < 1e-6f) continue;
                        fn(st, j, djx, djy, djz, r, rho_j);
                    }
                }
            }
        }
    }
}

typedef struct {
    float h, mass, gas_constant, rest_density, spiky_grad_coeff, p_i;
    float ax, ay, az;
} pressure_state;

/* sph_pressure.rs:86-99 */
static void pressure_pair(void* v, uint32_t j, float djx, float djy, float djz, float r,
                          float rho_j) {
    pressure_state* st = (pressure_state*)v;
    (void)j;
    float diff = st->h - r;
    float p_j = st->gas_constant * (rho_j - st->rest_density);
    float grad_scale = st->spiky_grad_coeff * diff * diff / r;
    float f_scale = -st->mass * (st->p_i + p_j) / (2.0f * rho_j) * grad_scale;
    st->ax += f_scale * djx;
    st->ay += f_scale * djy;
    st->az += f_scale * djz;
}

/* sph_pressure.rs:28-112 */
void or_sph_pressure(const or_sph_params* p, const float* px, const float* py, const float* pz,
                     const float* vx, const float* vy, const float* vz, const float* density,
                     uint32_t n, const uint32_t* cell_start, const uint32_t* sorted_indices,
                     float dt, float* vout) {
    float h2 = p->h * p->h;
    float h6 = h2 * h2 * h2;
    pressure_state st;
    st.h = p->h;
    st.mass = p->mass;
    st.gas_constant = p->gas_constant;
    st.rest_density = p->rest_density;
    st.spiky_grad_coeff = -45.0f / (3.14159265f * h6);
    for (uint32_t i = 0; i < n; i++) {
        float ox = vx[i], oy = vy[i], oz = vz[i];
        float rho_i = density[i];
        if (!(rho_i < 1e-6f)) { /* :42 -- early return leaves v_i untouched */
            st.p_i = p->gas_constant * (rho_i - p->rest_density);
            st.ax = st.ay = st.az = 0.0f;
            unfused_walk(p, px, py, pz, density, cell_start, sorted_indices, i, pressure_pair,
                         &st);
            ox += (st.ax / rho_i) * dt; /* :109-111 */
            oy += (st.ay / rho_i) * dt;
            oz += (st.az / rho_i) * dt;
        }
        vout[i] = ox;
        vout[(size_t)n + i] = oy;
        vout[2 * (size_t)n + i] = oz;
    }
}

typedef struct {
    float h, visc_coeff, mass, visc_lap_coeff, vxi, vyi, vzi;
    const float *vx, *vy, *vz;
    float ax, ay, az;
} viscosity_state;

/* sph_viscosity.rs:83-96 */
static void viscosity_pair(void* v, uint32_t j, float djx, float djy, float djz, float r,
                           float rho_j) {
    viscosity_state* st = (viscosity_state*)v;
    (void)djx;
    (void)djy;
    (void)djz;
    float lap = st->visc_lap_coeff * (st->h - r);
    float scale = st->visc_coeff * st->mass / rho_j * lap;
    st->ax += scale * (st->vx[j] - st->vxi);
    st->ay += scale * (st->vy[j] - st->vyi);
    st->az += scale * (st->vz[j] - st->vzi);
}

/* sph_viscosity.rs:27-106 */
void or_sph_viscosity(const or_sph_params* p, const float* px, const float* py,
                      const float* pz, const float* vx, const float* vy, const float* vz,
                      const float* density, uint32_t n, const uint32_t* cell_start,
                      const uint32_t* sorted_indices, float dt, float* vout) {
    float h2 = p->h * p->h;
    float h6 = h2 * h2 * h2;
    viscosity_state st;
    st.h = p->h;
    st.visc_coeff = p->visc;
    st.mass = p->mass;
    st.visc_lap_coeff = 45.0f / (3.14159265f * h6);
    st.vx = vx;
    st.vy = vy;
    st.vz = vz;
    for (uint32_t i = 0; i < n; i++) {
        float ox = vx[i], oy = vy[i], oz = vz[i];
        float rho_i = density[i];
        if (!(rho_i < 1e-6f)) { /* :42 */
            st.vxi = vx[i];
            st.vyi = vy[i];
            st.vzi = vz[i];
            st.ax = st.ay = st.az = 0.0f;
            unfused_walk(p, px, py, pz, density, cell_start, sorted_indices, i, viscosity_pair,
                         &st);
            ox += (st.ax / rho_i) * dt; /* :101-103 */
            oy += (st.ay / rho_i) * dt;
            oz += (st.az / rho_i) * dt;
        }
        vout[i] = ox;
        vout[(size_t)n + i] = oy;
        vout[2 * (size_t)n + i] = oz;
    }
}

/* gravity.rs:31-34 */
void or_gravity(float* vx, float* vy, float* vz, uint32_t n, float gx, float gy, float gz,
                float dt) {
    for (uint32_t i = 0; i < n; i++) {
        vx[i] += gx * dt;
        vy[i] += gy * dt;
        vz[i] += gz * dt;
    }
}

/* integrate.rs:16-31 */
void or_integrate(float* px, float* py, float* pz, float* vx, float* vy, float* vz, uint32_t n,
                  float dt) {
    for (uint32_t i = 0; i < n; i++) {
        float _vx = vx[i], _vy = vy[i], _vz = vz[i];
        if (!isfinite(_vx)) {
            _vx = 0.0f;
            vx[i] = 0.0f;
        }
        if (!isfinite(_vy)) {
            _vy = 0.0f;
            vy[i] = 0.0f;
        }
        if (!isfinite(_vz)) {
            _vz = 0.0f;
            vz[i] = 0.0f;
        }
        px[i] += _vx * dt;
        py[i] += _vy * dt;
        pz[i] += _vz * dt;
    }
}

/* box_collider.rs:26-47 */
void or_box_collider(float* px, float* py, float* pz, float* vx, float* vy, float* vz,
                     uint32_t n, const float mn[3], const float mx[3], float restitution) {
    float* p[3] = {px, py, pz};
    float* v[3] = {vx, vy, vz};
    for (uint32_t i = 0; i < n; i++)
        for (int c = 0; c < 3; c++) {
            if (p[c][i] < mn[c]) {
                p[c][i] = mn[c];
                v[c][i] = fabsf(v[c][i]) * restitution;
            }
            if (p[c][i] > mx[c]) {
                p[c][i] = mx[c];
                v[c][i] = -fabsf(v[c][i]) * restitution;
            }
        }
}

/* Pipeline::step (modules/mod.rs:98-104) over build_pipeline's order. */
int or_sph_step(const or_sph_params* p, uint32_t epi_flags, const float g[3], const float mn[3],
                const float mx[3], float restitution, float* px, float* py, float* pz,
                float* vx, float* vy, float* vz, uint32_t n, float dt, float* density,
                float* accel) {
    const float origin[3] = {0.0f, 0.0f, 0.0f};
    uint32_t C = p->dims[0] * p->dims[1] * p->dims[2];
    uint32_t* cell_start = (uint32_t*)malloc(((size_t)C + 1) * 4);
    uint32_t* sorted = (uint32_t*)malloc((size_t)(n ? n : 1) * 4);
    uint32_t* cells = (uint32_t*)malloc((size_t)(n ? n : 1) * 4);
    float* vout = (float*)malloc((size_t)(n ? n : 1) * 12);
    if (!cell_start || !sorted || !cells || !vout) {
        free(cell_start);
        free(sorted);
        free(cells);
        free(vout);
        return -1;
    }
    or_hashgrid_build(px, py, pz, 1, n, p->cell_size, origin, p->dims, cell_start, sorted, cells);
    or_sph_density(p, px, py, pz, n, cell_start, sorted, density);
    or_sph_force(p, px, py, pz, vx, vy, vz, density, n, cell_start, sorted, dt, vout, accel);
    memcpy(vx, vout, (size_t)n * 4);
    memcpy(vy, vout + n, (size_t)n * 4);
    memcpy(vz, vout + 2 * (size_t)n, (size_t)n * 4);
    if (epi_flags & 1u) or_gravity(vx, vy, vz, n, g[0], g[1], g[2], dt);
    if (epi_flags & 2u) or_integrate(px, py, pz, vx, vy, vz, n, dt);
    if (epi_flags & 4u) or_box_collider(px, py, pz, vx, vy, vz, n, mn, mx, restitution);
    free(cell_start);
    free(sorted);
    free(cells);
    free(vout);
    return 0;
}
