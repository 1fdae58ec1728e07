/*
 * forge_hip.h -- C ABI of the MI355X (gfx950) SPH / hash-grid hot path.
 *
 * This is the drop-in boundary that forge-gpu's host code would bind over FFI in place of its
 * NVRTC-compiled CUDA kernels.  Every entry point takes plain device pointers and sizes; the
 * caller owns every particle, key and output buffer, the context owns scratch, the stream and
 * the captured graph.
 *
 * Conventions
 *  - Return value: 0 = ok, < 0 = invalid argument (FH_E*), > 0 = a hipError_t code.
 *    Nothing aborts or unwinds across the ABI.  fh_last_error() returns a thread-local message
 *    describing the last failure on the calling thread.
 *  - All compute calls are asynchronous on the context stream (fh_stream()); fh_sync() waits.
 *    Results in caller buffers are visible after fh_sync() or any later work ordered on the
 *    same stream.
 *  - All scratch is allocated by fh_create(), so every compute call below is legal inside
 *    stream capture (no allocation, no memset node, no host synchronisation).
 *  - A context is used by one host thread at a time; several contexts may coexist.
 *  - "Position" inputs are three float pointers plus an element stride in floats, so both the
 *    structure-of-arrays layout of FieldSet (pos_x/pos_y/pos_z, stride 1) and the 12-byte
 *    Vec3f array-of-structures layout of HashGrid::build (x = p, y = p + 1, z = p + 2,
 *    stride 3) are accepted without a copy.
 *
 * Reference interfaces replaced (huaying/forge-gpu, paths relative to the repository root):
 *  - forge-runtime/src/hashgrid.rs:21-193      HashGrid::{new, build, position_to_cell, query_neighbors}
 *  - forge-runtime/src/radix_sort.rs:26-220    RadixSorter::{new, sort}
 *  - forge-runtime/src/radix_sort.rs:229-317   find_cell_boundaries
 *  - forge-manifest/src/modules/builtins/sph_density.rs:16-501   SphDensityModule::execute
 *  - forge-manifest/src/modules/builtins/sph_fused.rs:14-733     SphFusedModule::execute
 *  - forge-manifest/src/modules/builtins/sph_pressure.rs:9-161   SphPressureModule::execute
 *  - forge-manifest/src/modules/builtins/sph_viscosity.rs:9-155  SphViscosityModule::execute
 *  - forge-manifest/src/modules/builtins/gravity.rs:23-63        GravityModule::execute
 *  - forge-manifest/src/modules/builtins/integrate.rs:9-70       IntegrateModule::execute
 *  - forge-manifest/src/modules/builtins/box_collider.rs:18-85   BoxColliderModule::execute
 *  - forge-manifest/src/manifest_runner.rs:53-77                 graph capture / replay of substeps
 *  - forge-runtime/src/cuda.rs:55-63                             the simulation stream
 *  - forge-runtime/src/error.rs:7-22                             ForgeError (mapped to return codes)
 */
#ifndef FORGE_HIP_H
#define FORGE_HIP_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FH_ABI_VERSION 3

/* ---- status codes (negative: argument errors detected on the host) ------------------------- */
#define FH_OK 0
#define FH_EINVAL -1       /* null pointer, zero-sized grid, bad num_bits, ...                   */
#define FH_ERANGE -2       /* n > max_n or num_cells > max_cells of the context                 */
#define FH_ESTATE -3       /* call not legal in the current state (e.g. graph_end w/o begin)     */
#define FH_ENODEV -4       /* no HIP device, or the device is not gfx950                        */

typedef struct fh_ctx fh_ctx;

/* Parameters of the SPH passes.  Mirrors the fields of SphFusedModule
 * (forge-manifest/src/modules/builtins/sph_fused.rs:14-22); SphDensityModule uses the first
 * four (sph_density.rs:16-21).  The grid origin is (0,0,0), as in the reference kernels
 * (sph_fused.rs:91-93 hash with floorf(p / cell_size)). */
typedef struct fh_sph_params {
    float smoothing_radius;      /* h                                                       */
    float cell_size;             /* cs                                                      */
    uint32_t grid_dims[3];       /* nx, ny, nz                                              */
    float particle_mass;         /* m                                                       */
    float gas_constant;          /* k   (p = k (rho - rho0))                                */
    float rest_density;          /* rho0                                                    */
    float viscosity_coefficient; /* mu                                                      */
} fh_sph_params;

/* Epilogue of one substep, applied after the SPH velocity update in the order of
 * build_pipeline (manifest_runner.rs:371-393,508,528-537): gravity, integrate, box. */
#define FH_EPI_GRAVITY 1u
#define FH_EPI_INTEGRATE 2u
#define FH_EPI_BOX 4u
typedef struct fh_epilogue {
    uint32_t flags;              /* OR of FH_EPI_*                                          */
    float gravity[3];            /* GravityModule{gx,gy,gz}          (gravity.rs:5-9)       */
    float box_min[3];            /* BoxColliderModule{min_*}         (box_collider.rs:6-14) */
    float box_max[3];            /* BoxColliderModule{max_*}                                */
    float restitution;           /* BoxColliderModule::restitution                          */
} fh_epilogue;

/* ---- context -------------------------------------------------------------------------------- */

/* Create a context on HIP device `device` for up to `max_n` (<= 2^30, else FH_ERANGE)
 * particles / sort pairs and `max_cells` grid cells.  `stream` is an existing hipStream_t to run on, or NULL to create a
 * private default-priority stream.  Allocates every scratch buffer up front (replaces the lazy
 * scratch creation of sph_fused.rs:43-74 and RadixSorter::new, radix_sort.rs:55-70). */
int fh_create(int device, uint32_t max_n, uint32_t max_cells, void* stream, fh_ctx** out);
int fh_destroy(fh_ctx* ctx);
void* fh_stream(fh_ctx* ctx);                 /* the hipStream_t all calls are queued on       */
int fh_sync(fh_ctx* ctx);                     /* hipStreamSynchronize (Pipeline::step sync,
                                                 forge-manifest/src/modules/mod.rs:98-104)     */
const char* fh_last_error(void);              /* thread-local, never NULL                      */
int fh_abi_version(void);
/* Bytes of device scratch the context holds (for capacity planning). */
size_t fh_scratch_bytes(const fh_ctx* ctx);

/* ---- hashing -------------------------------------------------------------------------------- */

/* keys[i] = cell of particle i, vals[i] = i.  Cell: c = floor((p - origin) / cs) with Rust
 * `as i32` semantics (NaN -> 0, saturating), clamped to [0, dim-1], linearised
 * cx + cy*nx + cz*nx*ny (forge-runtime/src/hashgrid.rs:128-139; GPU twin without origin at
 * sph_fused.rs:84-100).  `vals` may be NULL. */
int fh_hash_cells(fh_ctx* ctx, const float* x, const float* y, const float* z, uint32_t stride,
                  uint32_t n, float cell_size, const float origin[3], const uint32_t dims[3],
                  uint32_t* keys, uint32_t* vals);

/* ---- sorting -------------------------------------------------------------------------------- */

/* Stable LSD radix sort of (key, value) pairs by the low `num_bits` bits of the key (1..32),
 * result in place in `keys`/`vals`.  Replaces RadixSorter::sort (radix_sort.rs:79-220), which
 * required num_bits % 4 == 0 and panicked on n > max_n; here any 1..32 is accepted and
 * n > max_n returns FH_ERANGE.  Equal keys keep their input order. */
int fh_sort_pairs(fh_ctx* ctx, uint32_t* keys, uint32_t* vals, uint32_t n, uint32_t num_bits);
/* The pass plan of the context's last sort (fh_sort_pairs, or the sort of a build / rebuild):
 * bit p set = digit pass p moved data; a pass whose digit is equal for every key is skipped
 * (for example the top byte of keys below 2^24).  No counterpart in the reference (whose every
 * 4-bit pass runs); for measurement.  Synchronises the stream. */
int fh_sort_plan(fh_ctx* ctx, uint32_t* plan);

/* fh_sort_pairs without a context, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  Same result as fh_sort_pairs (stable, in place, any 1..32 bits) for at most
 * FH_NOALLOC_MAX_N pairs (more: FH_ERANGE), queued on `stream` (NULL: the null stream) of the
 * current device.  All scratch is a fixed device array of FH_NOALLOC_SCRATCH_BYTES bytes in the
 * library, one copy per GPU held until the process ends; the call allocates nothing (the first
 * call on a device resolves the array's address).  Every call on one GPU shares that array:
 * calls ordered on one stream are fine, calls that overlap on one GPU (other streams, other
 * threads) race and must not be issued.  Errors: 0 / <0 / >0 as everywhere, message in
 * fh_last_error(). */
#define FH_NOALLOC_MAX_N 1048576u
#define FH_NOALLOC_SCRATCH_BYTES 19939328u
int fh_sort_pairs_noalloc(void* stream, uint32_t* keys, uint32_t* vals, uint32_t n,
                          uint32_t num_bits);
/* Device-side status of the no-alloc sorts on the current device: waits for `stream` (NULL: the
 * null stream), then reads and clears the device error flag of the fixed scratch.  FH_OK when
 * no no-alloc sort on this device gave up in a look-back since the last query (or none ran);
 * FH_ESTATE when one did (its output is wrong; fh_last_error() names the failure).  Like
 * fh_sync for a context, it is not legal during stream capture.  Allocates nothing (a 4-byte
 * copy each way). */
int fh_noalloc_status(void* stream);

/* From keys sorted ascending: cell_start[c] = first i with key c, cell_end[c] = last i + 1;
 * cells with no key keep cell_start = 0xFFFFFFFF, cell_end = 0.  Keys >= num_cells are
 * ignored.  Replaces find_cell_boundaries (radix_sort.rs:229-317, kernel :444-466). */
int fh_find_cell_boundaries(fh_ctx* ctx, const uint32_t* sorted_keys, uint32_t n,
                            uint32_t num_cells, uint32_t* cell_start, uint32_t* cell_end);

/* From keys sorted ascending: the CSR cell_start[0..C] with cell_start[c] = number of keys < c
 * (the exclusive prefix sum of the per-cell counts that HashGrid::build writes,
 * hashgrid.rs:102-106; cell_start[C] = n when every key is < C, keys >= C count in no cell).
 * C = num_cells (1..2^32-2); cell_start has C+1 words. */
int fh_cell_start_csr(fh_ctx* ctx, const uint32_t* sorted_keys, uint32_t n, uint32_t num_cells,
                      uint32_t* cell_start);

/* ---- hash grid ------------------------------------------------------------------------------ */

/* HashGrid::build on the GPU (hashgrid.rs:82-125): cell_indices[i] = cell of particle i,
 * cell_start[0..C] = exclusive prefix sum of the per-cell counts (cell_start[C] = n),
 * sorted_indices = particle ids ordered by cell, ascending id within a cell (the stable
 * counting-sort order of hashgrid.rs:109-117).  C = dims[0]*dims[1]*dims[2]. */
int fh_hashgrid_build(fh_ctx* ctx, const float* x, const float* y, const float* z,
                      uint32_t stride, uint32_t n, float cell_size, const float origin[3],
                      const uint32_t dims[3], uint32_t* cell_start, uint32_t* sorted_indices,
                      uint32_t* cell_indices);

/* For every point i of a grid built by fh_hashgrid_build over the same positions, count the
 * points j with ((dx*dx + dy*dy) + dz*dz) <= radius^2 (dx = p_j - p_i, self included, the
 * predicate and neighbourhood walk of HashGrid::query_neighbors, hashgrid.rs:145-193) and sum
 * their poly6 weights c*(r^2 - d^2)^3 with c = 315/(64*pi*r^9) (sph_density.rs:413-416 with
 * h = radius, no mass factor).  counts / wsum are in original point order; wsum may be NULL. */
int fh_neighbor_query(fh_ctx* ctx, const float* x, const float* y, const float* z,
                      uint32_t stride, uint32_t n, float cell_size, const float origin[3],
                      const uint32_t dims[3], const uint32_t* cell_start,
                      const uint32_t* sorted_indices, float radius, uint32_t* counts,
                      float* wsum);

/* HashGrid::query_neighbors (hashgrid.rs:145-193) for a batch of `nq` arbitrary query points
 * (qx/qy/qz with element stride qstride) against a grid built over the positions x/y/z.  The
 * query cell is not clamped; neighbours are visited in the reference's order (dz, dy, dx, then
 * cell order) and kept when ((dx*dx + dy*dy) + dz*dz) <= radius^2 with dx = p_j - q.
 * counts[q] receives the number of neighbours.  If `offsets` (nq+1 exclusive prefix sums of a
 * previous count call) and `indices` are non-NULL, the neighbour ids of query q are also
 * written to indices[offsets[q] .. offsets[q+1]). */
int fh_query_neighbors(fh_ctx* ctx, const float* x, const float* y, const float* z,
                       uint32_t stride, float cell_size, const float origin[3],
                       const uint32_t dims[3], const uint32_t* cell_start,
                       const uint32_t* sorted_indices, const float* qx, const float* qy,
                       const float* qz, uint32_t qstride, uint32_t nq, float radius,
                       uint32_t* counts, const uint32_t* offsets, uint32_t* indices);

/* ---- SPH modules ---------------------------------------------------------------------------- */

/* SphDensityModule::execute (sph_density.rs:388-501): rebuild the grid from pos and write
 * density[i] = sum over j in the 27-cell neighbourhood with r^2 < h^2 (self included) of
 * m * 315/(64*pi*h^9) * (h^2 - r^2)^3, in original particle order.  The reference module
 * leaves the rebuilt grid in the FieldSet's u32 fields (sph_density.rs:44-74), where the unfused
 * pressure / viscosity modules read it: when non-NULL, cell_start (C+1 words, CSR) and
 * sorted_indices (n words, ascending id within a cell) receive it here. */
int fh_sph_density(fh_ctx* ctx, const fh_sph_params* prm, const float* px, const float* py,
                   const float* pz, uint32_t n, float* density, uint32_t* cell_start,
                   uint32_t* sorted_indices);

/* SphPressureModule::execute (sph_pressure.rs:23-161): for each particle i with
 * rho_i >= 1e-6, a_p = sum over j != i of the 27-cell neighbourhood of the grid
 * (cell_start[C+1], sorted_indices[n] as written by fh_sph_density or fh_hashgrid_build with
 * origin 0) with r^2 < h^2, r^2 > 1e-12 and rho_j >= 1e-6 of
 * -m (p_i + p_j) / (2 rho_j) * (-45/(pi h^6)) (h - r)^2 / r * (x_i - x_j), p = k (rho - rho0);
 * then v_i += (a_p / rho_i) * dt in place.  Uses smoothing_radius, cell_size, grid_dims,
 * particle_mass, gas_constant and rest_density of prm. */
int fh_sph_pressure(fh_ctx* ctx, const fh_sph_params* prm, const float* px, const float* py,
                    const float* pz, float* vx, float* vy, float* vz, const float* density,
                    const uint32_t* cell_start, const uint32_t* sorted_indices, uint32_t n,
                    float dt);

/* SphViscosityModule::execute (sph_viscosity.rs:22-155): same neighbour set as
 * fh_sph_pressure; a_v = sum of mu m / rho_j * 45/(pi h^6) (h - r) * (v_j - v_i), every v_j
 * read from the velocities before this call (the reference kernel updates v in place while
 * other threads read it); then v_i += (a_v / rho_i) * dt.  Uses smoothing_radius, cell_size,
 * grid_dims, particle_mass and viscosity_coefficient of prm. */
int fh_sph_viscosity(fh_ctx* ctx, const fh_sph_params* prm, const float* px, const float* py,
                     const float* pz, float* vx, float* vy, float* vz, const float* density,
                     const uint32_t* cell_start, const uint32_t* sorted_indices, uint32_t n,
                     float dt);

/* SphFusedModule::execute (sph_fused.rs:413-732): rebuild, density, then the fused pressure +
 * viscosity pass: v_i += ((a_p + a_v) / rho_i) * dt, all neighbour velocities read from the
 * state before this call.  density (required) receives rho in original order; accel (may be
 * NULL) receives a_i = (a_p + a_v) / rho_i as 3 SoA arrays of n floats (accel, accel+n,
 * accel+2n).  If `epi` is non-NULL its flagged steps are fused into the force pass
 * (equivalent to running GravityModule, IntegrateModule and BoxColliderModule afterwards). */
int fh_sph_fused(fh_ctx* ctx, const fh_sph_params* prm, const fh_epilogue* epi, float* px,
                 float* py, float* pz, float* vx, float* vy, float* vz, float* density,
                 float* accel, uint32_t n, float dt);
/* The fused pressure + viscosity pass alone (the sph_fused_force kernel, sph_fused.rs:519-639,
 * as SphFusedModule::execute launches it after its rebuild and density pass, :700-726) over a
 * caller's grid and densities: cell_start[C+1] and sorted_indices[n] as fh_hashgrid_build or
 * fh_sph_density write them for these positions (origin 0), density[n] in particle order.
 * v_i += ((a_p + a_v) / rho_i) * dt in place, every neighbour velocity read from the state
 * before the call; accel (may be NULL) receives a_i as 3 SoA arrays of n floats.  Reference
 * expressions in the reference's neighbour order: bit-identical to the CPU restatement. */
int fh_sph_force(fh_ctx* ctx, const fh_sph_params* prm, const float* px, const float* py,
                 const float* pz, float* vx, float* vy, float* vz, const float* density,
                 const uint32_t* cell_start, const uint32_t* sorted_indices, float* accel,
                 uint32_t n, float dt);
/* `steps` (>= 1) consecutive fh_sph_fused substeps in one call, for a module that runs alone
 * in a pipeline's substep loop (Pipeline.run / capture, manifest_runner.rs:53-77, with
 * sph_fused.rs:413-732 each substep).  In the fast mode the state stays in HBM in cell-sorted
 * order between the substeps of the call: each later substep hashes and sorts the previous
 * substep's sorted state, and only the last one writes the caller's arrays (positions,
 * velocities, density, accel), so the arrays are not updated in between.  Particles of one cell
 * are then visited in the previous substep's order instead of ascending id, which changes sums
 * only by rounding.  With FH_OPT_SPH_EXACT, `steps` separate fh_sph_fused calls.
 * steps == 1 is fh_sph_fused. */
int fh_sph_fused_steps(fh_ctx* ctx, const fh_sph_params* prm, const fh_epilogue* epi, float* px,
                       float* py, float* pz, float* vx, float* vy, float* vz, float* density,
                       float* accel, uint32_t n, float dt, uint32_t steps);

/* Context options.  FH_OPT_SPH_EXACT = 1 makes fh_sph_density / fh_sph_fused evaluate the
 * reference's float expressions term by term in the reference's neighbour order (one thread per
 * particle, no FMA, IEEE division and square root: bit-identical to the CPU restatement, slower);
 * 0 (default) uses the LDS-tiled passes (fused multiply-adds, hardware reciprocal square root,
 * deterministic per-slab partial sums; within rel 1e-4). */
#define FH_OPT_SPH_EXACT 1
/* FH_OPT_HEAVY_WORK = 2: work split of the fast passes.  A (64-particle, z-slab) item whose
 * particles face more than `value` candidates (a co-located group counting as one) is processed
 * by 4 (or 8: FH_OPT_HEAVY_PARTS) wavefronts that split its candidates instead of one
 * wavefront; value 0 restores the default: 192, or 32 for calls of fewer than 2^18 particles,
 * whose few items would not fill the GPU otherwise.  Results differ only by rounding. */
#define FH_OPT_HEAVY_WORK 2
/* FH_OPT_DIRECT_ITEMS = 3: items whose particles' candidate ranges barely overlap (sparse
 * particles along a row, or beside a dense one) are walked transposed: one particle at a time,
 * its candidates across the lanes of a wavefront, instead of all particles through a
 * shared LDS-staged stream.  0: never, 1: chosen per item from the stream and per-particle
 * lengths (default), 2: every item.  Results differ only by rounding. */
#define FH_OPT_DIRECT_ITEMS 3
/* FH_OPT_HEAVY_PARTS = 4: wavefronts (4 or 8) that split each heavy item of the fast passes; 0
 * restores the default: 4, or 8 for calls of fewer than 2^18 particles where the context has
 * room for them.  More parts shorten the longest items (dense clumps: c4 is ~8 % faster with
 * 8) and give small systems more waves; fewer cost less per item (c3 is ~2 % faster with 4).
 * Results differ only by rounding.  A context of max_n >= 2^18 holds the parts' partial sums
 * for 4 parts; the first time 8 are set it makes room for 8 (one allocation, twice the
 * FH_OPT_HEAVY_SLOTS buffer below, so set it outside capture; fh_scratch_bytes counts it; the
 * context's captured graph is dropped and any graph captured on its stream before must be
 * captured again).  A smaller context has room for 8 from its creation. */
#define FH_OPT_HEAVY_PARTS 4
/* FH_OPT_EPOCH_PERIOD = 5: the work tags of the SPH rebuilds (co-located groups, skipped
 * sub-tiles, candidate group cells) compare a 30-bit epoch that every sort / rebuild start
 * bumps on the device, so a tag left 2^30 - 1 starts earlier would match again.  The context
 * counts the starts it queues (graph replays included) and, before the count reaches the
 * period, queues a renewal (tags cleared, epoch back to 0) between two calls or replays.
 * value = the period in starts (1..2^30 - 2; 0 restores the default 2^30 - 2); setting it
 * renews at once.  Short periods exercise the renewal in tests; results do not change. */
#define FH_OPT_EPOCH_PERIOD 5
/* FH_OPT_SPIN_LIMIT = 6 (diagnostics): polls a radix-sort look-back walk makes before it gives
 * up and raises the device error flag that fh_sync reports (0 restores the default, 2^22, far
 * above what any walk needs).  A limit of 1 forces that failure path without a fault (every
 * walk that needs a second poll gives up; the scatter stays in bounds, the output is wrong and
 * fh_sync returns FH_ESTATE).  Synchronises the stream. */
#define FH_OPT_SPIN_LIMIT 6
/* FH_OPT_HEAVY_SLOTS = 7: partial-sum slots of the fast passes' heavy items (4 KB each with 4
 * parts, 8 KB with 8).  By default a context of max_n >= 2^18 has one per 8 (64-particle,
 * z-slab) items of max_n (24 bytes per particle with 4 parts; a slot per item would take 192),
 * a smaller context one per item.  A heavy item that gets no slot in a substep is walked by one
 * wavefront, part after part, and its parts are added in the same order as a slotted item's:
 * the results are the same bit for bit, only that item is slower (workloads whose items are
 * mostly heavy, like dense clumps, want a slot per item).  value = slots (0 restores the
 * default; more than the items gives every item one).  One allocation, made at once: set it
 * outside capture; fh_scratch_bytes counts it; the context's captured graph is dropped and any
 * graph captured on its stream before must be captured again. */
#define FH_OPT_HEAVY_SLOTS 7
/* FH_OPT_SUBCELL = 8: sub-cells per axis (0: off, the default; 2, 4 or 8) by which the fused
 * module's fast rebuilds order the particles inside each cell (Morton order of the sub-cells:
 * 3, 6 or 9 more key bits, so more sort passes where the keys then need them).  A run of
 * consecutive candidates then covers a small box: the heavy items skip the 64-candidate chunks
 * with no candidate within h of their particles' box and pass only the near candidates of the
 * others to the pair loop.  Dense clumps gain (configs[4] with 8: 98 -> 63 ms); moderate
 * densities lose more in the extra sort passes than they gain (configs[3]: 414 -> 425 us with
 * 2).  Results differ only by rounding (the summation order); fh_sph_density and the bit-exact
 * mode are not affected. */
#define FH_OPT_SUBCELL 8
int fh_set_option(fh_ctx* ctx, int option, int value);

/* GravityModule (gravity.rs:31-34): v += g * dt. */
int fh_gravity(fh_ctx* ctx, float* vx, float* vy, float* vz, uint32_t n, float gx, float gy,
               float gz, float dt);
/* IntegrateModule (integrate.rs:16-31): non-finite velocity components are zeroed (and
 * stored), then p += v * dt. */
int fh_integrate(fh_ctx* ctx, float* px, float* py, float* pz, float* vx, float* vy,
                 float* vz, uint32_t n, float dt);
/* BoxColliderModule (box_collider.rs:26-47): per axis, p < min -> (p = min, v = |v| e), then
 * p > max -> (p = max, v = -|v| e). */
int fh_box_collider(fh_ctx* ctx, float* px, float* py, float* pz, float* vx, float* vy,
                    float* vz, uint32_t n, const float box_min[3], const float box_max[3],
                    float restitution);

/* ---- frames (run_manifest_streaming, manifest_runner.rs:145-167; serve.rs:7-10,43-62) ------- */

/* Pack the binary position frame of the streaming runner into the device buffer `out`
 * (8 + 12 n bytes, 4-byte aligned): u32 frame number, u32 particle count n, then
 * x0 y0 z0 x1 y1 z1 ... as f32, all little-endian.  The frame number is `frame`, or, when
 * frame_counter (a device u32) is non-NULL, the counter's value, which the call then
 * increments on the device -- so a captured graph that packs a frame emits consecutive
 * numbers on its replays.  Copying `out` to the host is the caller's (one contiguous D2H). */
int fh_pack_frame(fh_ctx* ctx, const float* px, const float* py, const float* pz, uint32_t n,
                  uint32_t frame, uint32_t* frame_counter, void* out);

/* ---- graphs (run_manifest capture/replay, manifest_runner.rs:53-77) ------------------------- */

/* Begin capturing the context stream; every fh_* compute call until fh_graph_end is recorded
 * instead of run.  fh_graph_end instantiates (replacing any previous graph of this context);
 * fh_graph_launch replays it `count` times on the context stream. */
int fh_graph_begin(fh_ctx* ctx);
int fh_graph_end(fh_ctx* ctx);
int fh_graph_launch(fh_ctx* ctx, uint32_t count);

/* ---- timing of the launches on the context stream ------------------------------------------ */

/* Record a HIP event on the context stream into slot `slot` (0..15); fh_event_elapsed_ms gives
 * the time between two recorded slots after they completed. */
int fh_event_record(fh_ctx* ctx, uint32_t slot);
int fh_event_elapsed_ms(fh_ctx* ctx, uint32_t slot_start, uint32_t slot_end, float* ms);

/* Per-kernel timing.  Arm kernel `name` (one of "hist", "hash", "scan", "sort",
 * "gather", "density", "force", "query", "finalize", "plan", "prep", "epoch_reset";
 * or a whole fast pass of fh_sph_fused, "density_pass" or "force_pass", from its first launch
 * to its last) so
 * that its next
 * `max_launches` launches on the
 * context stream are bracketed by HIP events; launches captured into a graph record the events
 * on every replay.  max_launches = 0 disarms.  Arming allocates events: call outside capture.
 * fh_kernel_times waits for the last armed launch and writes the durations (ms) of the armed
 * launches made so far (up to `cap`) into ms[], their number into *count. */
int fh_time_kernel(fh_ctx* ctx, const char* name, uint32_t max_launches);
int fh_kernel_times(fh_ctx* ctx, const char* name, float* ms, uint32_t cap, uint32_t* count);

#ifdef __cplusplus
}
#endif

#endif /* FORGE_HIP_H */
