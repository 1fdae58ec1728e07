/*
 * oracle.h -- CPU restatement of forge-gpu's SPH / hash-grid path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP path: it may be linked or
 * called only by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg.  The
 * product library (libforge_hip.so) never calls it and has no CPU fallback.
 *
 * Plain C11, single-threaded, built with -O2 -ffp-contract=off (no FMA contraction, no fast
 * math), so every float expression is evaluated exactly as written, in the order written, as
 * Rust (which never contracts) evaluates the reference's CPU code.
 *
 * Each function cites the reference file:line it restates (paths relative to the reference
 * repository root).  How each function is pinned (golden vectors from the reference's tests,
 * library cross-checks, closed forms, brute force) is listed in tests/test_oracle.py.
 */
#ifndef FORGE_ORACLE_H
#define FORGE_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Rust `f32 as i32`: NaN -> 0, saturating at i32::MIN / i32::MAX, else truncation. */
int32_t or_f32_as_i32(float f);

/* HashGrid::position_to_cell, forge-runtime/src/hashgrid.rs:128-139. */
uint32_t or_position_to_cell(float x, float y, float z, float cell_size, const float origin[3],
                             const uint32_t dims[3]);

/* Hash loop of HashGrid::build, hashgrid.rs:89-92; vals[i] = i (may be NULL). */
void or_hash_cells(const float* x, const float* y, const float* z, uint32_t stride, uint32_t n,
                   float cell_size, const float origin[3], const uint32_t dims[3],
                   uint32_t* keys, uint32_t* vals);

/* Stable sort of (key, val) pairs by the low num_bits bits of the key: the order that
 * RadixSorter::sort must produce (radix_sort.rs:79-220) and that the reference test compares
 * against with the stable `sort_by_key` (tests/radix_sort_test.rs:111-127).  Bottom-up merge
 * sort.  Returns 0, or -1 on allocation failure / bad num_bits. */
int or_stable_sort_pairs(uint32_t* keys, uint32_t* vals, uint32_t n, uint32_t num_bits);

/* find_cell_boundaries, radix_sort.rs:229-317 + kernel :444-466.  Keys >= num_cells skipped. */
void or_find_cell_boundaries(const uint32_t* sorted_keys, uint32_t n, uint32_t num_cells,
                             uint32_t* cell_start, uint32_t* cell_end);

/* CSR cell ranges from sorted keys: cell_start[c] = #keys < c for c in 0..C (length C+1);
 * keys >= C are not counted (hashgrid.rs:95-106). */
void or_cell_start_csr(const uint32_t* sorted_keys, uint32_t n, uint32_t num_cells,
                       uint32_t* cell_start);

/* HashGrid::build, hashgrid.rs:82-125 (count, exclusive scan, stable scatter). */
int or_hashgrid_build(const float* x, const float* y, const float* z, uint32_t stride,
                      uint32_t n, float cell_size, const float origin[3], const uint32_t dims[3],
                      uint32_t* cell_start, uint32_t* sorted_indices, uint32_t* cell_indices);

/* HashGrid::query_neighbors, hashgrid.rs:145-193.  Writes up to `cap` indices to `out` in
 * visiting order, returns the number of neighbours found (which may exceed cap). */
uint32_t or_query_neighbors(float qx, float qy, float qz, float radius, const float* x,
                            const float* y, const float* z, uint32_t stride, float cell_size,
                            const float origin[3], const uint32_t dims[3],
                            const uint32_t* cell_start, const uint32_t* sorted_indices,
                            uint32_t* out, uint32_t cap);

/* Every point as a query of its own grid: counts[i] = |query_neighbors(p_i, radius)| and
 * wsum[i] = sum of c*(r^2 - d^2)^3 over those neighbours, c = 315/(64*pi*r^9)
 * (sph_density.rs:413-416, h = radius, mass factor 1), summed in visiting order. */
void or_neighbor_counts(const float* x, const float* y, const float* z, uint32_t stride,
                        uint32_t n, float cell_size, const float origin[3],
                        const uint32_t dims[3], const uint32_t* cell_start,
                        const uint32_t* sorted_indices, float radius, uint32_t* counts,
                        float* wsum);

/* SPH parameters (SphFusedModule fields, sph_fused.rs:14-22). */
typedef struct or_sph_params {
    float h, cell_size;
    uint32_t dims[3];
    float mass, gas_constant, rest_density, visc;
} or_sph_params;

/* Untiled SPH density kernel, sph_density.rs:401-461, one particle at a time in index order.
 * Grid (cell_start, sorted_indices) as built by or_hashgrid_build with origin 0. */
void or_sph_density(const or_sph_params* p, const float* px, const float* py, const float* pz,
                    uint32_t n, const uint32_t* cell_start, const uint32_t* sorted_indices,
                    float* density);

/* or_sph_density for the particles which[0..m) only: density[k] of particle which[k], the
 * same per-particle sum in the same order (for workloads too large for the full pass). */
void or_sph_density_at(const or_sph_params* p, const float* px, const float* py,
                       const float* pz, const uint32_t* cell_start,
                       const uint32_t* sorted_indices, const uint32_t* which, uint32_t m,
                       float* density);

/* Fused pressure + viscosity pass, per-pair maths of sph_fused.rs:542-638 over the true
 * 27-cell neighbourhood, every neighbour velocity read from the input state (vx..vz are not
 * modified).  Writes vout = v + a*dt (if non-NULL) and accel a = (a_p + a_v)/rho_i (if non-NULL),
 * each as 3 arrays of n floats. */
void or_sph_force(const or_sph_params* p, const float* px, const float* py, const float* pz,
                  const float* vx, const float* vy, const float* vz, const float* density,
                  uint32_t n, const uint32_t* cell_start, const uint32_t* sorted_indices,
                  float dt, float* vout, float* accel);

/* fp64 restatement of or_sph_force (same neighbour set, selected with the fp32 r^2 tests):
 * accel64 = a_i in double, scale64 = sum_j (|pressure term| + |viscosity term|) / rho_i per
 * component -- the error scale of the force tolerance -- and, if sens64 is non-NULL,
 * sens64 = sum_j |d(pressure term + viscosity term)/dr| * 8 * 2^-24 * r / rho_i (per term, the
 * change an 8-unit float32 rounding of the pair distance makes: the factor h - r cancels near
 * r = h, so such a rounding moves the term by far more than 2^-24 of itself). */
void or_sph_force_f64(const or_sph_params* p, const float* px, const float* py,
                      const float* pz, const float* vx, const float* vy, const float* vz,
                      const float* density, uint32_t n, const uint32_t* cell_start,
                      const uint32_t* sorted_indices, double* accel64, double* scale64,
                      double* sens64);

/* or_sph_force_f64 for the particles which[0..m) only: accel64 / scale64 / sens64 as 3 arrays
 * of m doubles, entry k for particle which[k]. */
void or_sph_force_f64_at(const or_sph_params* p, const float* px, const float* py,
                         const float* pz, const float* vx, const float* vy, const float* vz,
                         const float* density, const uint32_t* cell_start,
                         const uint32_t* sorted_indices, const uint32_t* which, uint32_t m,
                         double* accel64, double* scale64, double* sens64);

/* Unfused SphPressureModule kernel, sph_pressure.rs:28-112: for each particle i with
 * rho_i >= 1e-6, a_p over the 27-cell neighbourhood of the grid (cell_start, sorted_indices as
 * left by the density module), skipping j == i, pairs with r^2 < h^2 && r^2 > 1e-12 and
 * rho_j >= 1e-6; then v_i += (a_p / rho_i) * dt.  Reads vx..vz and writes vout (3 arrays of n
 * floats); velocities are not read by the pressure terms. */
void or_sph_pressure(const or_sph_params* p, const float* px, const float* py, const float* pz,
                     const float* vx, const float* vy, const float* vz, const float* density,
                     uint32_t n, const uint32_t* cell_start, const uint32_t* sorted_indices,
                     float dt, float* vout);

/* Unfused SphViscosityModule kernel, sph_viscosity.rs:27-106: a_v = sum_j mu*m/rho_j *
 * lap(h - r) * (v_j - v_i) over the same neighbour set as or_sph_pressure, every v_j read from
 * the input state (the reference kernel updates v in place while neighbours read it; the
 * intended semantics is the state before the pass); then v_i += (a_v / rho_i) * dt into vout. */
void or_sph_viscosity(const or_sph_params* p, const float* px, const float* py,
                      const float* pz, const float* vx, const float* vy, const float* vz,
                      const float* density, uint32_t n, const uint32_t* cell_start,
                      const uint32_t* sorted_indices, float dt, float* vout);

/* GravityModule kernel, gravity.rs:31-34. */
void or_gravity(float* vx, float* vy, float* vz, uint32_t n, float gx, float gy, float gz,
                float dt);
/* IntegrateModule kernel, integrate.rs:16-31. */
void or_integrate(float* px, float* py, float* pz, float* vx, float* vy, float* vz, uint32_t n,
                  float dt);
/* BoxColliderModule kernel, box_collider.rs:26-47. */
void or_box_collider(float* px, float* py, float* pz, float* vx, float* vy, float* vz,
                     uint32_t n, const float mn[3], const float mx[3], float restitution);

/* One Pipeline::step of build_pipeline's order (manifest_runner.rs:334-393,508,528-537):
 * fused SPH (rebuild + density + force), then gravity / integrate / box per `epi_flags`
 * (1 gravity, 2 integrate, 4 box).  State arrays are updated in place; density and accel
 * (3n floats, may be NULL) receive the SPH outputs.  Returns 0, or -1 on allocation failure. */
int or_sph_step(const or_sph_params* p, uint32_t epi_flags, const float g[3], const float mn[3],
                const float mx[3], float restitution, float* px, float* py, float* pz,
                float* vx, float* vy, float* vz, uint32_t n, float dt, float* density,
                float* accel);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_ORACLE_H */
