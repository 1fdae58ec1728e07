// fh_api.hip -- the extern "C" boundary (include/forge_hip.h): argument checks, context and
// scratch ownership, the stream, graph capture and the orchestration of the kernels in
// fh_sort.hip, fh_grid.hip and fh_sph.hip.  No CPU fallback: every compute entry point
// enqueues HIP kernels or fails with a status code.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "fh_internal.hpp"

using namespace fh;

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* where) {
    return fail((int)e, "%s: %s (%d)", where, hipGetErrorString(e), (int)e);
}

#define FH_CHECK_HIP(expr)                                  \
    do {                                                    \
        hipError_t e_ = (expr);                             \
        if (e_ != hipSuccess) return hip_fail(e_, #expr);   \
    } while (0)

int check_ctx(fh_ctx* c) {
    if (!c) return fail(FH_EINVAL, "null context");
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    return FH_OK;
}

int check_n(fh_ctx* c, uint32_t n, const char* what) {
    if (n > c->max_n) return fail(FH_ERANGE, "%s: n=%u exceeds max_n=%u", what, n, c->max_n);
    return FH_OK;
}

// Validates a grid description and returns its cell count in *cells.
int check_grid(fh_ctx* c, float cs, const float* origin, const uint32_t* dims, GridDesc* g,
               uint32_t* cells, const char* what) {
    if (!dims) return fail(FH_EINVAL, "%s: null dims", what);
    if (!(cs > 0.0f) || cs != cs || cs > 3.0e38f)
        return fail(FH_EINVAL, "%s: cell_size must be finite and > 0", what);
    uint64_t C = 1;
    for (int q = 0; q < 3; q++) {
        if (dims[q] == 0 || dims[q] > (1u << 24))
            return fail(FH_EINVAL, "%s: grid dim %d = %u outside 1..2^24", what, q, dims[q]);
        C *= dims[q];
    }
    if (C > 0xFFFFFFFFull) return fail(FH_EINVAL, "%s: grid has more than 2^32-1 cells", what);
    if (C > c->max_cells)
        return fail(FH_ERANGE, "%s: %llu cells exceed max_cells=%u", what,
                    (unsigned long long)C, c->max_cells);
    g->cs = cs;
    g->ox = origin ? origin[0] : 0.0f;
    g->oy = origin ? origin[1] : 0.0f;
    g->oz = origin ? origin[2] : 0.0f;
    g->nx = dims[0];
    g->ny = dims[1];
    g->nz = dims[2];
    g->div_x = make_divu32(dims[0]);
    g->div_xy = make_divu32(dims[0] * dims[1]);
    g->sb = 0u;
    *cells = (uint32_t)C;
    return FH_OK;
}

int check_sph(fh_ctx* c, const fh_sph_params* p, GridDesc* g, uint32_t* cells, const char* what) {
    if (!p) return fail(FH_EINVAL, "%s: null params", what);
    if (!(p->smoothing_radius > 0.0f)) return fail(FH_EINVAL, "%s: smoothing_radius <= 0", what);
    static const float zero[3] = {0.0f, 0.0f, 0.0f};
    return check_grid(c, p->cell_size, zero, p->grid_dims, g, cells, what);
}

template <typename T>
hipError_t alloc(T** p, size_t count, size_t* total) {
    size_t bytes = count * sizeof(T);
    if (bytes == 0) bytes = sizeof(T);
    *total += bytes;
    return hipMalloc((void**)p, bytes);
}

// Partial-sum slots of a context by default: one per item below kSmallSystemN particles (whose
// default splits every heavy item 8 ways; a few MB), else one per kDefaultSlotShare items, 24
// bytes per particle of max_n with 4 parts (configs[3]'s trajectory numbers fewer than 4,096 of
// its 49,152 items' slots; a heavy item past the slots is walked part after part by one wave,
// with the same results).
constexpr uint32_t kDefaultSlotShare = 8;
static uint32_t default_slots(const fh_ctx* c) {
    return c->max_n < kSmallSystemN
               ? kHeavyLists * c->heavy_cap
               : kHeavyLists * ceil_div(c->heavy_cap, kDefaultSlotShare);
}

// Rebuild of the SPH grid from the positions: hash + digit histograms, the stable sort giving
// skeys / sidx (ascending id within a cell) and rank (its inverse), the gather into sorted
// float4 order, and the CSR cell_start from the sorted keys (with the candidate co-located
// groups of the fast passes).
// g.sb > 0 (the fused module's fast path): the keys carry the sub-cell below the cell
// (sort_key_of), and the last sort pass drops it, so skeys holds cells.
hipError_t sph_rebuild(fh_ctx* c, const GridDesc& g, uint32_t cells, const float* px,
                       const float* py, const float* pz, const float* vx, const float* vy,
                       const float* vz, uint32_t n, bool with_vel) {
    const uint32_t bits = bits_for_cells(cells) + g.sb;
    hipError_t e = launch_hash_hist(c, px, py, pz, 1, n, g, bits, c->kb, nullptr, true);
    if (e == hipSuccess && n > 0)
        e = launch_sort_passes(c, c->kb, nullptr, c->skeys, c->sidx, n, bits, c->rank, g.sb);
    if (e == hipSuccess)
        e = launch_gather(c, g, cells, px, py, pz, vx, vy, vz, n, with_vel, !c->sph_exact);
    return e;
}

// The same from the previous substep's new state in sorted order (c->sout), whose slots take
// the place of particle ids as sort values; its cells were written to c->kb by the previous
// substep's k_finalize, so only their histograms remain to be counted.
hipError_t sph_rebuild_resident(fh_ctx* c, const GridDesc& g, uint32_t cells, uint32_t n) {
    const uint32_t bits = bits_for_cells(cells) + g.sb;
    hipError_t e = n ? launch_hist_keys(c, c->kb, n, bits, true) : hipSuccess;
    if (e == hipSuccess && n > 0)
        e = launch_sort_passes(c, c->kb, nullptr, c->skeys, c->sidx2, n, bits, nullptr, g.sb);
    if (e == hipSuccess) e = launch_gather_resident(c, cells, n);
    return e;
}

}  // namespace

namespace fh {
// Epoch renewal: every tag array back to "untagged" (0) and the epoch to 0, so the next start
// makes it 1 again.  Queued by the host between starts (never captured).
__global__ __launch_bounds__(256) void k_epoch_reset(Control* ctl, uint64_t* run_tag,
                                                     uint64_t* cell_grp, uint32_t cells,
                                                     uint32_t* skip_tag, uint32_t subs) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < cells; i += stride) {
        run_tag[i] = 0ull;
        cell_grp[i] = 0ull;
    }
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < subs; i += stride)
        skip_tag[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x == 0) ctl->epoch = 0u;
}

static hipError_t launch_epoch_reset(fh_ctx* c) {
    uint32_t blocks = ceil_div(c->max_cells, 256u * 4u);
    if (blocks > 2048u) blocks = 2048u;
    if (blocks < 1u) blocks = 1u;
    tbeg(c, KID_EPOCH);
    k_epoch_reset<<<blocks, 256, 0, c->stream>>>(c->ctl, c->run_tag, c->cell_grp, c->max_cells,
                                                 c->skip_tag, ceil_div(c->max_n, 64u));
    tend(c, KID_EPOCH);
    return hipGetLastError();
}

hipError_t note_begin(fh_ctx* c) {
    if (!c->epoch_period) return hipSuccess;
    if (c->capturing) {  // replays are counted by fh_graph_launch
        c->capture_begins++;
        return hipSuccess;
    }
    if (c->begins + 1u > c->epoch_period) {
        const hipError_t e = launch_epoch_reset(c);
        if (e != hipSuccess) return e;
        c->begins = 0;
    }
    c->begins++;
    return hipSuccess;
}

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace fh

extern "C" {

int fh_abi_version(void) { return FH_ABI_VERSION; }

const char* fh_last_error(void) { return g_err; }

int fh_create(int device, uint32_t max_n, uint32_t max_cells, void* stream, fh_ctx** out) {
    if (!out) return fail(FH_EINVAL, "fh_create: null out");
    *out = nullptr;
    if (max_n == 0 || max_cells == 0) return fail(FH_EINVAL, "fh_create: max_n and max_cells must be > 0");
    if (max_n > kMaxSortN)
        return fail(FH_ERANGE, "fh_create: max_n=%u exceeds the supported 2^30", max_n);
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0)
        return fail(FH_ENODEV, "fh_create: no HIP device");
    if (device < 0 || device >= count) return fail(FH_ENODEV, "fh_create: no device %d", device);
    hipDeviceProp_t prop;
    FH_CHECK_HIP(hipGetDeviceProperties(&prop, device));
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(FH_ENODEV, "fh_create: device %d is %s, this library is built for gfx950",
                    device, prop.gcnArchName);
    FH_CHECK_HIP(hipSetDevice(device));

    fh_ctx* c = new fh_ctx();
    memset(c, 0, sizeof(*c));
    c->device = device;
    c->max_n = max_n;
    c->max_cells = max_cells;
    c->direct_mode = 1u;
    c->epoch_period = kEpochPeriod;
    c->max_sort_tiles = ceil_div(max_n, (uint32_t)kSortTile);
    size_t tot = 0;
    hipError_t e = hipSuccess;
    if (e == hipSuccess) e = alloc(&c->ka, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->va, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->kb, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->vb, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->sort_lb, (size_t)c->max_sort_tiles * kDigitSlots, &tot);
    // a histogram row per kHistChunk keys, at most kHistBlocks rows (the histogram kernels'
    // grid for a sort of n <= max_n keys)
    const uint32_t hist_rows =
        std::min(ceil_div(max_n, (uint32_t)kHistChunk), (uint32_t)kHistBlocks);
    if (e == hipSuccess) e = alloc(&c->hist_part, (size_t)hist_rows * kDigitSlots, &tot);
    // first-pass prefixes (sorts of up to kHistBlocks * kHistChunk keys): at most a tile per row
    // and a group sum per kHistRowsPerReduce / 2 tiles
    if (e == hipSuccess)
        e = alloc(&c->sort_pre,
                  ((size_t)hist_rows + ceil_div(hist_rows, (uint32_t)kHistRowsPerReduce / 2u)) * 1024u,
                  &tot);
    if (e == hipSuccess) e = alloc(&c->ctl, 1, &tot);
    if (e == hipSuccess) e = alloc(&c->run_tag, max_cells, &tot);
    if (e == hipSuccess) e = alloc(&c->cell_start, (size_t)max_cells + 1, &tot);
    if (e == hipSuccess) e = alloc(&c->skeys, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->sidx, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->spos, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->svel, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->srho, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->dpart, 3 * (size_t)max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->fpart, 9 * (size_t)max_n, &tot);
    // plan workgroup b appends to sub-list b % kHeavyLists, at most 3 * kPlanThreads / 64 items
    c->heavy_cap = 3u * (kPlanThreads / 64u) *
                   ceil_div(ceil_div(max_n, (uint32_t)kPlanThreads), (uint32_t)kHeavyLists);
    if (e == hipSuccess) e = alloc(&c->heavy, (size_t)kHeavyLists * c->heavy_cap, &tot);
    if (e == hipSuccess) e = alloc(&c->heavy_flag, 3 * (size_t)ceil_div(max_n, 64u), &tot);
    // partial sums of the heavy parts: default_slots() slots (FH_OPT_HEAVY_SLOTS sets them),
    // kHeavyWaves parts x kHeavyComps x 64 lanes each (room for kHeavyWavesMax parts is made
    // when FH_OPT_HEAVY_PARTS asks for it, and from the start for small contexts, whose default
    // is kHeavyWavesMax parts)
    c->hpart_parts = max_n < kSmallSystemN ? (uint32_t)kHeavyWavesMax : (uint32_t)kHeavyWaves;
    c->hslot_cap = default_slots(c);
    if (e == hipSuccess)
        e = alloc(&c->hpart, (size_t)c->hslot_cap * c->hpart_parts * kHeavyComps * 64u, &tot);
    if (e == hipSuccess) e = alloc(&c->hslot, 3 * (size_t)ceil_div(max_n, 64u), &tot);
    if (e == hipSuccess)
        e = alloc(&c->lstream, 3 * (size_t)ceil_div(max_n, 64u) * kLightCacheWords, &tot);
    if (e == hipSuccess) e = alloc(&c->lstream_t, 3 * (size_t)ceil_div(max_n, 64u), &tot);
    if (e == hipSuccess) e = alloc(&c->cell_grp, max_cells, &tot);
    if (e == hipSuccess) e = alloc(&c->big, (size_t)ceil_div(max_n, 64u) + 1u, &tot);
    if (e == hipSuccess) e = alloc(&c->skip_tag, (size_t)ceil_div(max_n, 64u), &tot);
    // the representatives' viscosity weights share the density partials' planes: the force
    // pass writes them after k_prep has read the last density partial, k_finalize reads them,
    // and a call that computes density only reads the partials and writes no weights
    c->wpart = c->dpart;
    if (e == hipSuccess) e = alloc(&c->vrep, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->rank, max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->sout, 3 * (size_t)max_n, &tot);
    if (e == hipSuccess) e = alloc(&c->sidx2, max_n, &tot);
    if (e == hipSuccess) e = hipHostMalloc((void**)&c->h_error, sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) {
        if (stream) {
            c->stream = (hipStream_t)stream;
        } else {
            e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
            c->own_stream = e == hipSuccess;
        }
    }
    // One-time clears (outside any capture): look-back words and run tags start untagged
    // (epoch 0 is never current).
    if (e == hipSuccess) e = hipMemsetAsync(c->sort_lb, 0, (size_t)c->max_sort_tiles * kDigitSlots * 4u, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->ctl, 0, sizeof(Control), c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->run_tag, 0, (size_t)max_cells * 8u, c->stream);
    if (e == hipSuccess) e = hipMemsetAsync(c->cell_grp, 0, (size_t)max_cells * 8u, c->stream);
    if (e == hipSuccess)
        e = hipMemsetAsync(c->skip_tag, 0, (size_t)ceil_div(max_n, 64u) * 4u, c->stream);
    for (int q = 0; q < kEvents && e == hipSuccess; q++) e = hipEventCreate(&c->ev[q]);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    c->scratch_bytes = tot;
    if (e != hipSuccess) {
        int rc = hip_fail(e, "fh_create");
        fh_destroy(c);
        return rc;
    }
    *out = c;
    return FH_OK;
}

int fh_destroy(fh_ctx* c) {
    if (!c) return FH_OK;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->exec) (void)hipGraphExecDestroy(c->exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    for (int q = 0; q < kEvents; q++)
        if (c->ev[q]) (void)hipEventDestroy(c->ev[q]);
    for (int k = 0; k < KID_COUNT; k++) {
        Timer& t = c->timers[k];
        if (t.ev) {
            for (uint32_t q = 0; q < 2 * t.max; q++)
                if (t.ev[q]) (void)hipEventDestroy(t.ev[q]);
            delete[] t.ev;
        }
    }
    void* bufs[] = {c->ka, c->va, c->kb, c->vb, c->sort_lb, c->ctl, c->run_tag,
                    c->cell_start, c->skeys, c->sidx, c->spos, c->svel,
                    c->srho, c->dpart, c->fpart, c->heavy, c->heavy_flag, c->hpart, c->hslot, c->lstream, c->lstream_t, c->hist_part,
                    c->sort_pre,
                    c->cell_grp, c->big, c->skip_tag, c->vrep, c->rank, c->sout,
                    c->sidx2};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (c->h_error) (void)hipHostFree(c->h_error);
    if (c->own_stream && c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return FH_OK;
}

void* fh_stream(fh_ctx* c) { return c ? (void*)c->stream : nullptr; }

size_t fh_scratch_bytes(const fh_ctx* c) { return c ? c->scratch_bytes : 0; }

int fh_sync(fh_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (c->capturing) return fail(FH_ESTATE, "fh_sync: stream is being captured");
    FH_CHECK_HIP(hipMemcpyAsync(c->h_error, &c->ctl->error.v, sizeof(uint32_t),
                                hipMemcpyDeviceToHost, c->stream));
    FH_CHECK_HIP(hipStreamSynchronize(c->stream));
    if (*c->h_error) {
        uint32_t code = *c->h_error;
        FH_CHECK_HIP(hipMemsetAsync(&c->ctl->error.v, 0, sizeof(uint32_t), c->stream));
        FH_CHECK_HIP(hipStreamSynchronize(c->stream));
        return fail(FH_ESTATE, "fh_sync: device reported a look-back failure (code %u)", code);
    }
    return FH_OK;
}

int fh_hash_cells(fh_ctx* c, const float* x, const float* y, const float* z, uint32_t stride,
                  uint32_t n, float cell_size, const float origin[3], const uint32_t dims[3],
                  uint32_t* keys, uint32_t* vals) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!keys || (n && (!x || !y || !z)) || stride == 0)
        return fail(FH_EINVAL, "fh_hash_cells: null pointer or zero stride");
    GridDesc g;
    uint32_t cells;
    if ((rc = check_grid(c, cell_size, origin, dims, &g, &cells, "fh_hash_cells"))) return rc;
    if (n == 0) return FH_OK;
    FH_CHECK_HIP(launch_hash_hist(c, x, y, z, stride, n, g, 0, keys, vals, false));
    return FH_OK;
}

int fh_sort_pairs(fh_ctx* c, uint32_t* keys, uint32_t* vals, uint32_t n, uint32_t num_bits) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && (!keys || !vals)) return fail(FH_EINVAL, "fh_sort_pairs: null keys or values");
    if (num_bits < 1 || num_bits > 32)
        return fail(FH_EINVAL, "fh_sort_pairs: num_bits=%u outside 1..32", num_bits);
    if ((rc = check_n(c, n, "fh_sort_pairs"))) return rc;
    if (n < 2) return FH_OK;
    FH_CHECK_HIP(launch_hist_keys(c, keys, n, num_bits, true));
    // In place: the last pass that runs writes the caller's buffers (see sort_plan).
    FH_CHECK_HIP(launch_sort_passes(c, keys, vals, keys, vals, n, num_bits));
    return FH_OK;
}

int fh_sort_plan(fh_ctx* c, uint32_t* plan) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!plan) return fail(FH_EINVAL, "fh_sort_plan: null output");
    if (c->capturing) return fail(FH_ESTATE, "fh_sort_plan: stream is being captured");
    FH_CHECK_HIP(hipMemcpyAsync(c->h_error, &c->ctl->plan, sizeof(uint32_t),
                                hipMemcpyDeviceToHost, c->stream));
    FH_CHECK_HIP(hipStreamSynchronize(c->stream));
    *plan = *c->h_error;
    return FH_OK;
}

int fh_find_cell_boundaries(fh_ctx* c, const uint32_t* sorted_keys, uint32_t n,
                            uint32_t num_cells, uint32_t* cell_start, uint32_t* cell_end) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((n && !sorted_keys) || !cell_start || !cell_end)
        return fail(FH_EINVAL, "fh_find_cell_boundaries: null pointer");
    if (num_cells == 0) return fail(FH_EINVAL, "fh_find_cell_boundaries: num_cells == 0");
    FH_CHECK_HIP(launch_boundaries(c, sorted_keys, n, num_cells, cell_start, cell_end));
    return FH_OK;
}

int fh_cell_start_csr(fh_ctx* c, const uint32_t* sorted_keys, uint32_t n, uint32_t num_cells,
                      uint32_t* cell_start) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if ((n && !sorted_keys) || !cell_start)
        return fail(FH_EINVAL, "fh_cell_start_csr: null pointer");
    if (num_cells == 0 || num_cells == 0xFFFFFFFFu)
        return fail(FH_EINVAL, "fh_cell_start_csr: num_cells must be in 1..2^32-2");
    FH_CHECK_HIP(launch_csr_from_sorted(c, sorted_keys, n, num_cells, cell_start));
    return FH_OK;
}

int fh_hashgrid_build(fh_ctx* c, const float* x, const float* y, const float* z,
                      uint32_t stride, uint32_t n, float cell_size, const float origin[3],
                      const uint32_t dims[3], uint32_t* cell_start, uint32_t* sorted_indices,
                      uint32_t* cell_indices) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!cell_start || (n && (!x || !y || !z || !sorted_indices || !cell_indices)) || stride == 0)
        return fail(FH_EINVAL, "fh_hashgrid_build: null pointer or zero stride");
    if ((rc = check_n(c, n, "fh_hashgrid_build"))) return rc;
    GridDesc g;
    uint32_t cells;
    if ((rc = check_grid(c, cell_size, origin, dims, &g, &cells, "fh_hashgrid_build"))) return rc;
    const uint32_t bits = bits_for_cells(cells);
    FH_CHECK_HIP(launch_hash_hist(c, x, y, z, stride, n, g, bits, cell_indices, nullptr, true));
    if (n > 0)
        FH_CHECK_HIP(launch_sort_passes(c, cell_indices, nullptr, c->skeys, sorted_indices, n, bits));
    // CSR straight from the sorted keys (each run start fills the empty cells before it): no
    // count, no scan
    tbeg(c, KID_SCAN);
    const hipError_t e = launch_csr_from_sorted(c, c->skeys, n, cells, cell_start);
    tend(c, KID_SCAN);
    FH_CHECK_HIP(e);
    return FH_OK;
}

int fh_neighbor_query(fh_ctx* c, const float* x, const float* y, const float* z,
                      uint32_t stride, uint32_t n, float cell_size, const float origin[3],
                      const uint32_t dims[3], const uint32_t* cell_start,
                      const uint32_t* sorted_indices, float radius, uint32_t* counts,
                      float* wsum) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!cell_start || (n && (!x || !y || !z || !sorted_indices || !counts)) || stride == 0)
        return fail(FH_EINVAL, "fh_neighbor_query: null pointer or zero stride");
    if ((rc = check_n(c, n, "fh_neighbor_query"))) return rc;
    if (!(radius >= 0.0f)) return fail(FH_EINVAL, "fh_neighbor_query: radius must be >= 0");
    GridDesc g;
    uint32_t cells;
    if ((rc = check_grid(c, cell_size, origin, dims, &g, &cells, "fh_neighbor_query"))) return rc;
    FH_CHECK_HIP(launch_neighbor_query(c, x, y, z, stride, n, g, cell_start, sorted_indices,
                                       radius, counts, wsum));
    return FH_OK;
}

int fh_query_neighbors(fh_ctx* c, const float* x, const float* y, const float* z,
                       uint32_t stride, float cell_size, const float origin[3],
                       const uint32_t dims[3], const uint32_t* cell_start,
                       const uint32_t* sorted_indices, const float* qx, const float* qy,
                       const float* qz, uint32_t qstride, uint32_t nq, float radius,
                       uint32_t* counts, const uint32_t* offsets, uint32_t* indices) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!x || !y || !z || !cell_start || !sorted_indices || stride == 0 || qstride == 0 ||
        (nq && (!qx || !qy || !qz || !counts)))
        return fail(FH_EINVAL, "fh_query_neighbors: null pointer or zero stride");
    if ((offsets == nullptr) != (indices == nullptr))
        return fail(FH_EINVAL, "fh_query_neighbors: offsets and indices go together");
    if (!(radius >= 0.0f)) return fail(FH_EINVAL, "fh_query_neighbors: radius must be >= 0");
    GridDesc g;
    uint32_t cells;
    if ((rc = check_grid(c, cell_size, origin, dims, &g, &cells, "fh_query_neighbors"))) return rc;
    FH_CHECK_HIP(launch_query(c, x, y, z, stride, g, cell_start, sorted_indices, qx, qy, qz,
                              qstride, nq, radius, counts, offsets, indices));
    return FH_OK;
}

int fh_sph_density(fh_ctx* c, const fh_sph_params* prm, const float* px, const float* py,
                   const float* pz, uint32_t n, float* density, uint32_t* cell_start,
                   uint32_t* sorted_indices) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && (!px || !py || !pz || !density)) return fail(FH_EINVAL, "fh_sph_density: null pointer");
    if ((rc = check_n(c, n, "fh_sph_density"))) return rc;
    GridDesc g;
    uint32_t cells;
    if ((rc = check_sph(c, prm, &g, &cells, "fh_sph_density"))) return rc;
    FH_CHECK_HIP(sph_rebuild(c, g, cells, px, py, pz, nullptr, nullptr, nullptr, n, false));
    // the grid as rebuilt (ascending id within a cell), before the fast passes regroup cells
    FH_CHECK_HIP(launch_copy_grid(c, cells, n, cell_start, sorted_indices));
    if (n == 0) return FH_OK;
    SphArgs a{g, prm->smoothing_radius, prm->particle_mass, prm->gas_constant,
              prm->rest_density, prm->viscosity_coefficient, 0.0f, n};
    if (c->sph_exact) {
        FH_CHECK_HIP(launch_density(c, a, c->cell_start, density));
    } else {
        FH_CHECK_HIP(launch_group_plan(c, a, false));
        FH_CHECK_HIP(launch_density_fast(c, a, c->cell_start));
        FH_CHECK_HIP(launch_finalize(c, a, nullptr, true, nullptr, nullptr, nullptr, nullptr,
                                     nullptr, nullptr, density, nullptr));
    }
    return FH_OK;
}

// `steps` substeps of the fused SPH step.  The first rebuilds from the caller's arrays; in the
// fast mode the later ones start from the previous substep's new state, kept in sorted order
// (resident), and only the last moves its state to the caller's arrays.
static int sph_fused_steps(fh_ctx* c, const fh_sph_params* prm, const fh_epilogue* epi,
                           float* px, float* py, float* pz, float* vx, float* vy, float* vz,
                           float* density, float* accel, uint32_t n, float dt, uint32_t steps,
                           const char* what) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && (!px || !py || !pz || !vx || !vy || !vz || !density))
        return fail(FH_EINVAL, "%s: null pointer", what);
    if (steps == 0) return fail(FH_EINVAL, "%s: steps must be >= 1", what);
    if ((rc = check_n(c, n, what))) return rc;
    if (epi && (epi->flags & ~(FH_EPI_GRAVITY | FH_EPI_INTEGRATE | FH_EPI_BOX)))
        return fail(FH_EINVAL, "%s: unknown epilogue flags 0x%x", what, epi->flags);
    GridDesc g;
    uint32_t cells;
    if ((rc = check_sph(c, prm, &g, &cells, what))) return rc;
    // FH_OPT_SUBCELL: the fast rebuilds order each cell by sub-cell (keys that still fit 32 bits)
    if (!c->sph_exact && bits_for_cells(cells) + c->sub_bits <= 32u) g.sb = c->sub_bits;
    SphArgs a{g, prm->smoothing_radius, prm->particle_mass, prm->gas_constant,
              prm->rest_density, prm->viscosity_coefficient, dt, n};
    for (uint32_t k = 0; k < steps; k++) {
        const bool resident = k > 0 && !c->sph_exact && n > 0;
        const bool last = k + 1 == steps || c->sph_exact;
        if (resident)
            FH_CHECK_HIP(sph_rebuild_resident(c, g, cells, n));
        else
            FH_CHECK_HIP(sph_rebuild(c, g, cells, px, py, pz, vx, vy, vz, n, true));
        if (n == 0) continue;
        if (c->sph_exact) {
            FH_CHECK_HIP(launch_density(c, a, c->cell_start, density));
            FH_CHECK_HIP(launch_force(c, a, epi, c->cell_start, px, py, pz, vx, vy, vz, accel));
            continue;
        }
        FH_CHECK_HIP(launch_group_plan(c, a, true));
        // pass timers: wall time of each pass (the force pass with its k_prep)
        tbeg(c, KID_DPASS);
        FH_CHECK_HIP(launch_density_fast(c, a, c->cell_start));
        tend(c, KID_DPASS);
        tbeg(c, KID_FPASS);
        FH_CHECK_HIP(launch_prep(c, a));
        FH_CHECK_HIP(launch_force_fast(c, a, c->cell_start));
        tend(c, KID_FPASS);
        FH_CHECK_HIP(launch_finalize(c, a, epi, false, px, py, pz, vx, vy, vz, density,
                                     last ? accel : nullptr, last, last && steps > 1,
                                     last ? nullptr : c->kb));
    }
    return FH_OK;
}

int fh_sph_fused(fh_ctx* c, const fh_sph_params* prm, const fh_epilogue* epi, float* px,
                 float* py, float* pz, float* vx, float* vy, float* vz, float* density,
                 float* accel, uint32_t n, float dt) {
    return sph_fused_steps(c, prm, epi, px, py, pz, vx, vy, vz, density, accel, n, dt, 1u,
                           "fh_sph_fused");
}

int fh_sph_fused_steps(fh_ctx* c, const fh_sph_params* prm, const fh_epilogue* epi, float* px,
                       float* py, float* pz, float* vx, float* vy, float* vz, float* density,
                       float* accel, uint32_t n, float dt, uint32_t steps) {
    return sph_fused_steps(c, prm, epi, px, py, pz, vx, vy, vz, density, accel, n, dt, steps,
                           "fh_sph_fused_steps");
}

int fh_sph_force(fh_ctx* c, const fh_sph_params* prm, const float* px, const float* py,
                 const float* pz, float* vx, float* vy, float* vz, const float* density,
                 const uint32_t* cell_start, const uint32_t* sorted_indices, float* accel,
                 uint32_t n, float dt) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!cell_start || (n && (!px || !py || !pz || !vx || !vy || !vz || !density || !sorted_indices)))
        return fail(FH_EINVAL, "fh_sph_force: null pointer");
    if ((rc = check_n(c, n, "fh_sph_force"))) return rc;
    GridDesc g;
    uint32_t cells;
    if ((rc = check_sph(c, prm, &g, &cells, "fh_sph_force"))) return rc;
    if (n == 0) return FH_OK;
    SphArgs a{g, prm->smoothing_radius, prm->particle_mass, prm->gas_constant,
              prm->rest_density, prm->viscosity_coefficient, dt, n};
    // the caller's state in the caller's grid order, then the exact fused pass (velocities
    // written back through sorted_indices; positions untouched without an epilogue)
    FH_CHECK_HIP(launch_gather_grid(c, px, py, pz, vx, vy, vz, density, sorted_indices, n));
    FH_CHECK_HIP(launch_force(c, a, nullptr, cell_start, nullptr, nullptr, nullptr, vx, vy, vz,
                              accel));
    return FH_OK;
}

int fh_pack_frame(fh_ctx* c, const float* px, const float* py, const float* pz, uint32_t n,
                  uint32_t frame, uint32_t* frame_counter, void* out) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!out || (n && (!px || !py || !pz))) return fail(FH_EINVAL, "fh_pack_frame: null pointer");
    if (n > (0xFFFFFFFFu - 2u) / 3u)
        return fail(FH_ERANGE, "fh_pack_frame: n=%u does not fit a frame", n);
    FH_CHECK_HIP(launch_pack_frame(c, px, py, pz, n, frame, frame_counter, out));
    return FH_OK;
}

static int unfused(fh_ctx* c, bool viscosity, const fh_sph_params* prm, const float* px,
                   const float* py, const float* pz, float* vx, float* vy, float* vz,
                   const float* density, const uint32_t* cell_start,
                   const uint32_t* sorted_indices, uint32_t n, float dt) {
    const char* what = viscosity ? "fh_sph_viscosity" : "fh_sph_pressure";
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!cell_start || (n && (!px || !py || !pz || !vx || !vy || !vz || !density || !sorted_indices)))
        return fail(FH_EINVAL, "%s: null pointer", what);
    if ((rc = check_n(c, n, what))) return rc;
    GridDesc g;
    uint32_t cells;
    if ((rc = check_sph(c, prm, &g, &cells, what))) return rc;
    SphArgs a{g, prm->smoothing_radius, prm->particle_mass, prm->gas_constant,
              prm->rest_density, prm->viscosity_coefficient, dt, n};
    FH_CHECK_HIP(launch_unfused(c, viscosity, a, px, py, pz, vx, vy, vz, density, cell_start,
                                sorted_indices));
    return FH_OK;
}

int fh_sph_pressure(fh_ctx* c, const fh_sph_params* prm, const float* px, const float* py,
                    const float* pz, float* vx, float* vy, float* vz, const float* density,
                    const uint32_t* cell_start, const uint32_t* sorted_indices, uint32_t n,
                    float dt) {
    return unfused(c, false, prm, px, py, pz, vx, vy, vz, density, cell_start, sorted_indices,
                   n, dt);
}

int fh_sph_viscosity(fh_ctx* c, const fh_sph_params* prm, const float* px, const float* py,
                     const float* pz, float* vx, float* vy, float* vz, const float* density,
                     const uint32_t* cell_start, const uint32_t* sorted_indices, uint32_t n,
                     float dt) {
    return unfused(c, true, prm, px, py, pz, vx, vy, vz, density, cell_start, sorted_indices,
                   n, dt);
}

// The heavy parts' partial-sum buffer for `slots` slots of `parts` parts each: one allocation
// (callers have checked that no capture is in progress), the old buffer freed after the stream
// has drained.  The context's captured graph holds the old buffer and slot count, so it is
// dropped (fh_graph_launch then fails with FH_ESTATE until a graph is captured again).
static int resize_hpart(fh_ctx* c, uint32_t slots, uint32_t parts) {
    const size_t words = (size_t)slots * parts * kHeavyComps * 64u;
    const size_t old_words = (size_t)c->hslot_cap * c->hpart_parts * kHeavyComps * 64u;
    FH_CHECK_HIP(hipStreamSynchronize(c->stream));
    if (c->exec) (void)hipGraphExecDestroy(c->exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->exec = nullptr;
    c->graph = nullptr;
    c->graph_begins = 0;
    float* p = nullptr;
    const hipError_t ae = hipMalloc((void**)&p, (words ? words : 1u) * sizeof(float));
    if (ae != hipSuccess) return hip_fail(ae, "fh_set_option: heavy part buffer");
    (void)hipFree(c->hpart);
    c->scratch_bytes = c->scratch_bytes - old_words * sizeof(float) + words * sizeof(float);
    c->hpart = p;
    c->hslot_cap = slots;
    c->hpart_parts = parts;
    return FH_OK;
}

int fh_set_option(fh_ctx* c, int option, int value) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (c->capturing) return fail(FH_ESTATE, "fh_set_option: stream is being captured");
    switch (option) {
        case FH_OPT_SPH_EXACT:
            c->sph_exact = value != 0;
            return FH_OK;
        case FH_OPT_HEAVY_WORK:
            if (value < 0) return fail(FH_EINVAL, "fh_set_option: heavy work %d < 0", value);
            c->heavy_work = (uint32_t)value;
            return FH_OK;
        case FH_OPT_DIRECT_ITEMS:
            if (value < 0 || value > 2)
                return fail(FH_EINVAL, "fh_set_option: direct items mode %d outside 0..2", value);
            c->direct_mode = (uint32_t)value;
            return FH_OK;
        case FH_OPT_HEAVY_PARTS:
            if (value != 0 && value != kHeavyWaves && value != kHeavyWavesMax)
                return fail(FH_EINVAL, "fh_set_option: heavy parts %d is not 0, %d or %d", value,
                            kHeavyWaves, kHeavyWavesMax);
            if ((uint32_t)value > c->hpart_parts) {
                // the partial sums of every slot for `value` parts: a larger buffer, made once
                // (outside capture, checked above)
                const int rc2 = resize_hpart(c, c->hslot_cap, (uint32_t)value);
                if (rc2) return rc2;
            }
            c->heavy_parts = (uint32_t)value;
            return FH_OK;
        case FH_OPT_HEAVY_SLOTS: {
            if (value < 0) return fail(FH_EINVAL, "fh_set_option: heavy slots %d < 0", value);
            const uint32_t all = kHeavyLists * c->heavy_cap;
            const uint32_t cap = value == 0              ? default_slots(c)
                                 : (uint32_t)value > all ? all
                                                         : (uint32_t)value;
            if (cap != c->hslot_cap) {
                const int rc2 = resize_hpart(c, cap, c->hpart_parts);
                if (rc2) return rc2;
            }
            return FH_OK;
        }
        case FH_OPT_SUBCELL:
            if (value != 0 && value != 2 && value != 4 && value != 8)
                return fail(FH_EINVAL, "fh_set_option: sub-cells per axis %d is not 0, 2, 4 or 8",
                            value);
            c->sub_bits = value == 8 ? 9u : value == 4 ? 6u : value == 2 ? 3u : 0u;
            return FH_OK;
        case FH_OPT_EPOCH_PERIOD:
            if (value < 0 || (uint32_t)value > kEpochPeriod)
                return fail(FH_EINVAL, "fh_set_option: epoch period %d outside 0..%u", value,
                            kEpochPeriod);
            c->epoch_period = value ? (uint32_t)value : kEpochPeriod;
            // renew now, so the count of the new period starts from the next start
            FH_CHECK_HIP(launch_epoch_reset(c));
            c->begins = 0;
            return FH_OK;
        case FH_OPT_SPIN_LIMIT: {
            if (value < 0) return fail(FH_EINVAL, "fh_set_option: spin limit %d < 0", value);
            const uint32_t v = (uint32_t)value;
            FH_CHECK_HIP(hipMemcpyAsync(&c->ctl->spin_limit, &v, sizeof(v), hipMemcpyHostToDevice,
                                        c->stream));
            FH_CHECK_HIP(hipStreamSynchronize(c->stream));
            return FH_OK;
        }
        default:
            return fail(FH_EINVAL, "fh_set_option: unknown option %d", option);
    }
}

int fh_gravity(fh_ctx* c, float* vx, float* vy, float* vz, uint32_t n, float gx, float gy,
               float gz, float dt) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && (!vx || !vy || !vz)) return fail(FH_EINVAL, "fh_gravity: null pointer");
    FH_CHECK_HIP(launch_gravity(c, vx, vy, vz, n, gx, gy, gz, dt));
    return FH_OK;
}

int fh_integrate(fh_ctx* c, float* px, float* py, float* pz, float* vx, float* vy, float* vz,
                 uint32_t n, float dt) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (n && (!px || !py || !pz || !vx || !vy || !vz))
        return fail(FH_EINVAL, "fh_integrate: null pointer");
    FH_CHECK_HIP(launch_integrate(c, px, py, pz, vx, vy, vz, n, dt));
    return FH_OK;
}

int fh_box_collider(fh_ctx* c, float* px, float* py, float* pz, float* vx, float* vy,
                    float* vz, uint32_t n, const float box_min[3], const float box_max[3],
                    float restitution) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!box_min || !box_max || (n && (!px || !py || !pz || !vx || !vy || !vz)))
        return fail(FH_EINVAL, "fh_box_collider: null pointer");
    FH_CHECK_HIP(launch_box(c, px, py, pz, vx, vy, vz, n, box_min, box_max, restitution));
    return FH_OK;
}

int fh_graph_begin(fh_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (c->capturing) return fail(FH_ESTATE, "fh_graph_begin: already capturing");
    FH_CHECK_HIP(hipStreamBeginCapture(c->stream, hipStreamCaptureModeRelaxed));
    c->capturing = true;
    c->capture_begins = 0;
    return FH_OK;
}

int fh_graph_end(fh_ctx* c) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!c->capturing) return fail(FH_ESTATE, "fh_graph_end: not capturing");
    c->capturing = false;
    hipGraph_t graph = nullptr;
    FH_CHECK_HIP(hipStreamEndCapture(c->stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipGraphInstantiate");
    }
    if (c->exec) (void)hipGraphExecDestroy(c->exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    c->graph = graph;
    c->exec = exec;
    c->graph_begins = c->capture_begins;
    c->capture_begins = 0;
    FH_CHECK_HIP(hipGraphUpload(c->exec, c->stream));
    return FH_OK;
}

int fh_graph_launch(fh_ctx* c, uint32_t count) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (!c->exec) return fail(FH_ESTATE, "fh_graph_launch: no captured graph");
    if (c->capturing) return fail(FH_ESTATE, "fh_graph_launch: stream is being captured");
    // Each replay starts graph_begins sorts / rebuilds: renew the epoch between replays before
    // the count since the last renewal would pass the period.
    for (uint32_t q = 0; q < count; q++) {
        if (c->epoch_period && c->graph_begins &&
            c->begins + c->graph_begins > c->epoch_period) {
            FH_CHECK_HIP(launch_epoch_reset(c));
            c->begins = 0;
        }
        FH_CHECK_HIP(hipGraphLaunch(c->exec, c->stream));
        c->begins += c->graph_begins;
    }
    return FH_OK;
}

int fh_event_record(fh_ctx* c, uint32_t slot) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (slot >= (uint32_t)kEvents) return fail(FH_EINVAL, "fh_event_record: slot %u", slot);
    FH_CHECK_HIP(hipEventRecord(c->ev[slot], c->stream));
    return FH_OK;
}

static const char* const kKernelNames[KID_COUNT] = {"hist", "hash", "scan", "sort",
                                                    "gather", "density", "force", "query",
                                                    "finalize", "plan", "prep",
                                                    "density_pass", "force_pass",
                                                    "epoch_reset"};

static int kernel_id(const char* name) {
    if (!name) return -1;
    for (int k = 0; k < KID_COUNT; k++)
        if (strcmp(name, kKernelNames[k]) == 0) return k;
    return -1;
}

static void free_timer(Timer& t) {
    if (t.ev) {
        for (uint32_t q = 0; q < 2 * t.max; q++)
            if (t.ev[q]) (void)hipEventDestroy(t.ev[q]);
        delete[] t.ev;
    }
    t.ev = nullptr;
    t.max = t.used = 0;
}

int fh_time_kernel(fh_ctx* c, const char* name, uint32_t max_launches) {
    int rc = check_ctx(c);
    if (rc) return rc;
    int k = kernel_id(name);
    if (k < 0) return fail(FH_EINVAL, "fh_time_kernel: unknown kernel '%s'", name ? name : "");
    if (c->capturing) return fail(FH_ESTATE, "fh_time_kernel: stream is being captured");
    if (max_launches > 4096) return fail(FH_EINVAL, "fh_time_kernel: at most 4096 launches");
    FH_CHECK_HIP(hipStreamSynchronize(c->stream));
    free_timer(c->timers[k]);
    if (max_launches == 0) return FH_OK;
    Timer& t = c->timers[k];
    t.ev = new hipEvent_t[2 * max_launches]();
    t.max = max_launches;
    for (uint32_t q = 0; q < 2 * max_launches; q++) {
        hipError_t e = hipEventCreate(&t.ev[q]);
        if (e != hipSuccess) {
            free_timer(t);
            return hip_fail(e, "hipEventCreate");
        }
    }
    return FH_OK;
}

int fh_kernel_times(fh_ctx* c, const char* name, float* ms, uint32_t cap, uint32_t* count) {
    int rc = check_ctx(c);
    if (rc) return rc;
    int k = kernel_id(name);
    if (k < 0 || !count || (cap && !ms)) return fail(FH_EINVAL, "fh_kernel_times: bad arguments");
    if (c->capturing) return fail(FH_ESTATE, "fh_kernel_times: stream is being captured");
    Timer& t = c->timers[k];
    uint32_t m = t.used < cap ? t.used : cap;
    if (t.used) FH_CHECK_HIP(hipEventSynchronize(t.ev[2 * t.used - 1]));
    for (uint32_t q = 0; q < m; q++)
        FH_CHECK_HIP(hipEventElapsedTime(&ms[q], t.ev[2 * q], t.ev[2 * q + 1]));
    *count = m;
    return FH_OK;
}

int fh_event_elapsed_ms(fh_ctx* c, uint32_t a, uint32_t b, float* ms) {
    int rc = check_ctx(c);
    if (rc) return rc;
    if (a >= (uint32_t)kEvents || b >= (uint32_t)kEvents || !ms)
        return fail(FH_EINVAL, "fh_event_elapsed_ms: bad slot or null output");
    if (c->capturing) return fail(FH_ESTATE, "fh_event_elapsed_ms: stream is being captured");
    FH_CHECK_HIP(hipEventSynchronize(c->ev[b]));
    FH_CHECK_HIP(hipEventElapsedTime(ms, c->ev[a], c->ev[b]));
    return FH_OK;
}

}  // extern "C"
