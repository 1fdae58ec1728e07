// forge_hip.hpp -- C++ host-side mirror of forge-gpu's interfaces for the SPH / hash-grid path,
// header-only, on top of the C ABI in forge_hip.h.
//
// The reference host code is Rust; its toolchain is not available here, so this header restates
// the same interfaces in C++ (same names, argument meaning and error behaviour) for C++ callers
// and for the parity tests that read like the reference's own tests:
//   forge::Array<T>              forge-runtime/src/array.rs:81-107,193-214,366-406 (device buffer,
//                                synchronous from_vec / to_vec)
//   forge::Error                 forge-runtime/src/error.rs:7-22 (thrown instead of Result::Err)
//   forge::HashGrid              forge-runtime/src/hashgrid.rs:21-193 (build runs on the GPU)
//   forge::RadixSorter           forge-runtime/src/radix_sort.rs:26-220
//   forge::find_cell_boundaries  forge-runtime/src/radix_sort.rs:229-317
//   forge::cell_start_csr        forge-runtime/src/hashgrid.rs:102-106 (from sorted keys)
//   forge::frame_bytes, pack_frame, Pipeline::run_streaming
//                                forge-manifest/src/manifest_runner.rs:145-181, serve.rs:7-10,43-62
//   forge::FieldSet, SimModule, Pipeline
//                                forge-manifest/src/modules/mod.rs:12-117
//   forge::SphFusedModule, SphDensityModule, SphPressureModule, SphViscosityModule,
//   GravityModule, IntegrateModule, BoxColliderModule
//                                forge-manifest/src/modules/builtins/{sph_fused,sph_density,
//                                sph_pressure,sph_viscosity,gravity,integrate,box_collider}.rs
// Exceptions stay on this side of the ABI: every C call returns a status that is turned into a
// forge::Error here.
#pragma once

#include <hip/hip_runtime_api.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "forge_hip.h"

namespace forge {

class Error : public std::runtime_error {
   public:
    Error(int code, const std::string& msg) : std::runtime_error(msg), code_(code) {}
    int code() const { return code_; }

   private:
    int code_;
};

inline void check(int rc) {
    if (rc != FH_OK) throw Error(rc, fh_last_error());
}

inline void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error((int)e, std::string(what) + ": " + hipGetErrorString(e));
}

// Owns an fh_ctx (stream + scratch), the counterpart of the reference's per-ordinal context and
// simulation stream (forge-runtime/src/cuda.rs:13-63).
class Context {
   public:
    Context(uint32_t max_n, uint32_t max_cells, int device = 0) {
        check(fh_create(device, max_n, max_cells, nullptr, &ctx_));
        max_n_ = max_n;
        max_cells_ = max_cells;
    }
    ~Context() {
        if (ctx_) fh_destroy(ctx_);
    }
    Context(const Context&) = delete;
    Context& operator=(const Context&) = delete;
    fh_ctx* get() const { return ctx_; }
    hipStream_t stream() const { return (hipStream_t)fh_stream(ctx_); }
    void sync() const { check(fh_sync(ctx_)); }
    uint32_t max_n() const { return max_n_; }
    uint32_t max_cells() const { return max_cells_; }

   private:
    fh_ctx* ctx_ = nullptr;
    uint32_t max_n_ = 0, max_cells_ = 0;
};

// Typed device buffer (Array<T>): RAII hipMalloc, synchronous host transfers.
template <typename T>
class Array {
   public:
    Array() = default;
    explicit Array(size_t n) : n_(n) {
        if (n) check_hip(hipMalloc((void**)&p_, n * sizeof(T)), "hipMalloc");
    }
    static Array zeros(size_t n) {
        Array a(n);
        if (n) check_hip(hipMemset(a.p_, 0, n * sizeof(T)), "hipMemset");
        return a;
    }
    static Array from_vec(const std::vector<T>& v) {
        Array a(v.size());
        if (!v.empty())
            check_hip(hipMemcpy(a.p_, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice),
                      "hipMemcpy");
        return a;
    }
    std::vector<T> to_vec() const {
        std::vector<T> v(n_);
        if (n_) check_hip(hipMemcpy(v.data(), p_, n_ * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
        return v;
    }
    ~Array() {
        if (p_) (void)hipFree(p_);
    }
    Array(Array&& o) noexcept : p_(o.p_), n_(o.n_) {
        o.p_ = nullptr;
        o.n_ = 0;
    }
    Array& operator=(Array&& o) noexcept {
        std::swap(p_, o.p_);
        std::swap(n_, o.n_);
        return *this;
    }
    Array(const Array&) = delete;
    Array& operator=(const Array&) = delete;
    T* data() { return p_; }
    const T* data() const { return p_; }
    size_t len() const { return n_; }

   private:
    T* p_ = nullptr;
    size_t n_ = 0;
};

struct Vec3f {  // forge-core Vec3f: #[repr(C)] 3 x f32, 12 bytes (forge-core/src/vec.rs:137-139)
    float x, y, z;
};
static_assert(sizeof(Vec3f) == 12, "Vec3f must be 12 bytes");

class HashGrid {
   public:
    HashGrid(Context& ctx, float cell_size, uint32_t dim_x, uint32_t dim_y, uint32_t dim_z,
             Vec3f origin, size_t max_particles)
        : ctx_(ctx), cell_size(cell_size), dim_x(dim_x), dim_y(dim_y), dim_z(dim_z),
          origin(origin), cell_start(Array<uint32_t>::zeros(num_cells() + 1)),
          sorted_indices(Array<uint32_t>::zeros(max_particles)),
          cell_indices(Array<uint32_t>::zeros(max_particles)) {}

    size_t num_cells() const { return (size_t)dim_x * dim_y * dim_z; }

    // Build from device-resident Vec3f positions (stride 3 floats).
    void build(const Array<Vec3f>& positions) {
        const size_t n = positions.len();
        if (n > sorted_indices.len()) {
            sorted_indices = Array<uint32_t>(n);
            cell_indices = Array<uint32_t>(n);
        }
        const float* p = reinterpret_cast<const float*>(positions.data());
        const float o[3] = {origin.x, origin.y, origin.z};
        const uint32_t d[3] = {dim_x, dim_y, dim_z};
        check(fh_hashgrid_build(ctx_.get(), p, p + 1, p + 2, 3, (uint32_t)n, cell_size, o, d,
                                cell_start.data(), sorted_indices.data(), cell_indices.data()));
        ctx_.sync();
        num_particles = n;
    }

    uint32_t position_to_cell(Vec3f pos) const {
        Array<Vec3f> p = Array<Vec3f>::from_vec({pos});
        Array<uint32_t> k(1);
        const float* f = reinterpret_cast<const float*>(p.data());
        const float o[3] = {origin.x, origin.y, origin.z};
        const uint32_t d[3] = {dim_x, dim_y, dim_z};
        check(fh_hash_cells(ctx_.get(), f, f + 1, f + 2, 3, 1, cell_size, o, d, k.data(), nullptr));
        ctx_.sync();
        return k.to_vec()[0];
    }

    // Neighbour ids of `pos` within `radius` (dist^2 <= r^2, visiting order of the reference).
    std::vector<uint32_t> query_neighbors(Vec3f pos, float radius,
                                          const Array<Vec3f>& positions) const {
        Array<Vec3f> q = Array<Vec3f>::from_vec({pos});
        Array<uint32_t> count(1), offsets = Array<uint32_t>::zeros(2);
        const float* p = reinterpret_cast<const float*>(positions.data());
        const float* qf = reinterpret_cast<const float*>(q.data());
        const float o[3] = {origin.x, origin.y, origin.z};
        const uint32_t d[3] = {dim_x, dim_y, dim_z};
        check(fh_query_neighbors(ctx_.get(), p, p + 1, p + 2, 3, cell_size, o, d, cell_start.data(),
                                 sorted_indices.data(), qf, qf + 1, qf + 2, 3, 1, radius,
                                 count.data(), nullptr, nullptr));
        ctx_.sync();
        const uint32_t c = count.to_vec()[0];
        std::vector<uint32_t> off = {0u, c};
        offsets = Array<uint32_t>::from_vec(off);
        Array<uint32_t> idx(c ? c : 1);
        check(fh_query_neighbors(ctx_.get(), p, p + 1, p + 2, 3, cell_size, o, d, cell_start.data(),
                                 sorted_indices.data(), qf, qf + 1, qf + 2, 3, 1, radius,
                                 count.data(), offsets.data(), idx.data()));
        ctx_.sync();
        std::vector<uint32_t> out = idx.to_vec();
        out.resize(c);
        return out;
    }

   private:
    Context& ctx_;

   public:
    float cell_size;
    uint32_t dim_x, dim_y, dim_z;
    Vec3f origin;
    Array<uint32_t> cell_start;
    Array<uint32_t> sorted_indices;
    Array<uint32_t> cell_indices;
    size_t num_particles = 0;
};

class RadixSorter {
   public:
    RadixSorter(Context& ctx, size_t max_n) : ctx_(ctx), max_n_(max_n) {}
    // Stable sort of (keys, values) by the low num_bits bits, in place.
    void sort(Array<uint32_t>& keys, Array<uint32_t>& values, size_t n, uint32_t num_bits) {
        if (n > max_n_) throw Error(FH_ERANGE, "n exceeds max_n");
        check(fh_sort_pairs(ctx_.get(), keys.data(), values.data(), (uint32_t)n, num_bits));
    }

   private:
    Context& ctx_;
    size_t max_n_;
};

inline void find_cell_boundaries(Context& ctx, const Array<uint32_t>& sorted_cell_ids,
                                 Array<uint32_t>& cell_start, Array<uint32_t>& cell_end, size_t n,
                                 size_t num_cells) {
    check(fh_find_cell_boundaries(ctx.get(), sorted_cell_ids.data(), (uint32_t)n,
                                  (uint32_t)num_cells, cell_start.data(), cell_end.data()));
}

// CSR cell ranges of cell keys the caller already sorted (the prefix sum of hashgrid.rs:102-106):
// cell_start[c] = number of keys < c for c = 0..num_cells; keys >= num_cells fall in no cell.
inline void cell_start_csr(Context& ctx, const Array<uint32_t>& sorted_keys, size_t n,
                           size_t num_cells, Array<uint32_t>& cell_start) {
    if (cell_start.len() < num_cells + 1)
        throw Error(FH_EINVAL, "cell_start needs num_cells + 1 entries");
    check(fh_cell_start_csr(ctx.get(), sorted_keys.data(), (uint32_t)n, (uint32_t)num_cells,
                            cell_start.data()));
}

// Named SoA particle fields in original particle order (modules/mod.rs:12-67).
class FieldSet {
   public:
    FieldSet(Context& ctx, size_t particle_count) : ctx(ctx), particle_count(particle_count) {}
    void add_f32(const std::string& name, const std::vector<float>& data) {
        f32_fields[name] = Array<float>::from_vec(data);
    }
    void add_f32_zeros(const std::string& name, size_t n) {
        f32_fields[name] = Array<float>::zeros(n);
    }
    Array<float>& f(const std::string& name) {
        auto it = f32_fields.find(name);
        if (it == f32_fields.end()) throw Error(FH_EINVAL, "missing field " + name);
        return it->second;
    }
    Array<uint32_t>& u(const std::string& name) {
        auto it = u32_fields.find(name);
        if (it == u32_fields.end()) throw Error(FH_EINVAL, "missing field " + name);
        return it->second;
    }
    Context& ctx;
    size_t particle_count;
    std::map<std::string, Array<float>> f32_fields;
    std::map<std::string, Array<uint32_t>> u32_fields;
};

class SimModule {
   public:
    virtual ~SimModule() = default;
    virtual const char* name() const = 0;
    // Creates the fields execute() writes but the caller may not have added (allocation and a
    // memset, so it must not run while a graph is being captured).
    virtual void prepare(FieldSet&) {}
    virtual void execute(FieldSet& fields, float dt) = 0;
};

struct SphFusedModule : SimModule {
    float smoothing_radius, cell_size;
    uint32_t grid_dims[3];
    float particle_mass, gas_constant, rest_density, viscosity_coefficient;
    bool has_epilogue = false;
    fh_epilogue epilogue{};
    SphFusedModule(float h, float cs, uint32_t nx, uint32_t ny, uint32_t nz, float m, float k,
                   float rho0, float mu)
        : smoothing_radius(h), cell_size(cs), grid_dims{nx, ny, nz}, particle_mass(m),
          gas_constant(k), rest_density(rho0), viscosity_coefficient(mu) {}
    const char* name() const override { return "sph_fused"; }
    void prepare(FieldSet& fs) override {
        if (!fs.f32_fields.count("density")) fs.add_f32_zeros("density", fs.particle_count);
    }
    void execute(FieldSet& fs, float dt) override {
        prepare(fs);
        const fh_sph_params p = params();
        check(fh_sph_fused(fs.ctx.get(), &p, has_epilogue ? &epilogue : nullptr,
                           fs.f("pos_x").data(), fs.f("pos_y").data(), fs.f("pos_z").data(),
                           fs.f("vel_x").data(), fs.f("vel_y").data(), fs.f("vel_z").data(),
                           fs.f("density").data(), nullptr, (uint32_t)fs.particle_count, dt));
    }
    // `steps` substeps in one call (fh_sph_fused_steps): the state stays on the device in
    // cell-sorted order between them and the fields are written after the last one.
    void execute_steps(FieldSet& fs, float dt, uint32_t steps) {
        prepare(fs);
        const fh_sph_params p = params();
        check(fh_sph_fused_steps(fs.ctx.get(), &p, has_epilogue ? &epilogue : nullptr,
                                 fs.f("pos_x").data(), fs.f("pos_y").data(), fs.f("pos_z").data(),
                                 fs.f("vel_x").data(), fs.f("vel_y").data(), fs.f("vel_z").data(),
                                 fs.f("density").data(), nullptr, (uint32_t)fs.particle_count, dt,
                                 steps));
    }
    // The fused force pass alone (sph_fused.rs:519-639) over the grid and densities that a
    // SphDensityModule left in the field set (u32 cell_start / sorted_indices, f32 density):
    // v += a dt in place; accel (3 n floats) receives a when non-null.
    void execute_force(FieldSet& fs, float dt, float* accel = nullptr) {
        const size_t cells = (size_t)grid_dims[0] * grid_dims[1] * grid_dims[2] + 1;
        if (fs.u("cell_start").len() != cells)
            throw Error(FH_EINVAL, "cell_start does not match the module's grid");
        const fh_sph_params p = params();
        check(fh_sph_force(fs.ctx.get(), &p, fs.f("pos_x").data(), fs.f("pos_y").data(),
                           fs.f("pos_z").data(), fs.f("vel_x").data(), fs.f("vel_y").data(),
                           fs.f("vel_z").data(), fs.f("density").data(), fs.u("cell_start").data(),
                           fs.u("sorted_indices").data(), accel, (uint32_t)fs.particle_count,
                           dt));
    }

   private:
    fh_sph_params params() const {
        return fh_sph_params{smoothing_radius, cell_size,
                             {grid_dims[0], grid_dims[1], grid_dims[2]},
                             particle_mass, gas_constant, rest_density, viscosity_coefficient};
    }
};

struct SphDensityModule : SimModule {
    float smoothing_radius, cell_size;
    uint32_t grid_dims[3];
    float particle_mass;
    SphDensityModule(float h, float cs, uint32_t nx, uint32_t ny, uint32_t nz, float m)
        : smoothing_radius(h), cell_size(cs), grid_dims{nx, ny, nz}, particle_mass(m) {}
    const char* name() const override { return "sph_density"; }
    // Also leaves its grid in the u32 fields cell_start / sorted_indices, which the unfused
    // pressure and viscosity modules read (sph_density.rs:44-74).
    void prepare(FieldSet& fs) override {
        if (!fs.f32_fields.count("density")) fs.add_f32_zeros("density", fs.particle_count);
        const size_t cells = (size_t)grid_dims[0] * grid_dims[1] * grid_dims[2] + 1;
        auto cs = fs.u32_fields.find("cell_start");
        if (cs == fs.u32_fields.end() || cs->second.len() != cells)
            fs.u32_fields["cell_start"] = Array<uint32_t>::zeros(cells);
        auto si = fs.u32_fields.find("sorted_indices");
        if (si == fs.u32_fields.end() || si->second.len() != fs.particle_count)
            fs.u32_fields["sorted_indices"] = Array<uint32_t>::zeros(fs.particle_count);
    }
    void execute(FieldSet& fs, float) override {
        prepare(fs);
        fh_sph_params p{smoothing_radius, cell_size, {grid_dims[0], grid_dims[1], grid_dims[2]},
                        particle_mass, 0.0f, 0.0f, 0.0f};
        check(fh_sph_density(fs.ctx.get(), &p, fs.f("pos_x").data(), fs.f("pos_y").data(),
                             fs.f("pos_z").data(), (uint32_t)fs.particle_count,
                             fs.f("density").data(), fs.u("cell_start").data(),
                             fs.u("sorted_indices").data()));
    }
};

// Unfused SphPressureModule (sph_pressure.rs:9-16) and SphViscosityModule
// (sph_viscosity.rs:9-15): read the density and grid fields SphDensityModule left behind.
struct SphPressureModule : SimModule {
    float gas_constant, rest_density, smoothing_radius, cell_size;
    uint32_t grid_dims[3];
    float particle_mass;
    SphPressureModule(float k, float rho0, float h, float cs, uint32_t nx, uint32_t ny,
                      uint32_t nz, float m)
        : gas_constant(k), rest_density(rho0), smoothing_radius(h), cell_size(cs),
          grid_dims{nx, ny, nz}, particle_mass(m) {}
    const char* name() const override { return "sph_pressure"; }
    void execute(FieldSet& fs, float dt) override {
        fh_sph_params p{smoothing_radius, cell_size, {grid_dims[0], grid_dims[1], grid_dims[2]},
                        particle_mass, gas_constant, rest_density, 0.0f};
        check(fh_sph_pressure(fs.ctx.get(), &p, fs.f("pos_x").data(), fs.f("pos_y").data(),
                              fs.f("pos_z").data(), fs.f("vel_x").data(), fs.f("vel_y").data(),
                              fs.f("vel_z").data(), fs.f("density").data(),
                              fs.u("cell_start").data(), fs.u("sorted_indices").data(),
                              (uint32_t)fs.particle_count, dt));
    }
};

struct SphViscosityModule : SimModule {
    float coefficient, smoothing_radius, cell_size;
    uint32_t grid_dims[3];
    float particle_mass;
    SphViscosityModule(float mu, float h, float cs, uint32_t nx, uint32_t ny, uint32_t nz,
                       float m)
        : coefficient(mu), smoothing_radius(h), cell_size(cs), grid_dims{nx, ny, nz},
          particle_mass(m) {}
    const char* name() const override { return "sph_viscosity"; }
    void execute(FieldSet& fs, float dt) override {
        fh_sph_params p{smoothing_radius, cell_size, {grid_dims[0], grid_dims[1], grid_dims[2]},
                        particle_mass, 0.0f, 0.0f, coefficient};
        check(fh_sph_viscosity(fs.ctx.get(), &p, fs.f("pos_x").data(), fs.f("pos_y").data(),
                               fs.f("pos_z").data(), fs.f("vel_x").data(), fs.f("vel_y").data(),
                               fs.f("vel_z").data(), fs.f("density").data(),
                               fs.u("cell_start").data(), fs.u("sorted_indices").data(),
                               (uint32_t)fs.particle_count, dt));
    }
};

struct GravityModule : SimModule {
    float gx, gy, gz;
    GravityModule(float gx, float gy, float gz) : gx(gx), gy(gy), gz(gz) {}
    static GravityModule default_earth() { return GravityModule(0.0f, -9.81f, 0.0f); }
    const char* name() const override { return "gravity"; }
    void execute(FieldSet& fs, float dt) override {
        check(fh_gravity(fs.ctx.get(), fs.f("vel_x").data(), fs.f("vel_y").data(),
                         fs.f("vel_z").data(), (uint32_t)fs.particle_count, gx, gy, gz, dt));
    }
};

struct IntegrateModule : SimModule {
    const char* name() const override { return "integrate"; }
    void execute(FieldSet& fs, float dt) override {
        check(fh_integrate(fs.ctx.get(), fs.f("pos_x").data(), fs.f("pos_y").data(),
                           fs.f("pos_z").data(), fs.f("vel_x").data(), fs.f("vel_y").data(),
                           fs.f("vel_z").data(), (uint32_t)fs.particle_count, dt));
    }
};

struct BoxColliderModule : SimModule {
    float min_x, min_y, min_z, max_x, max_y, max_z, restitution;
    BoxColliderModule(float x0, float y0, float z0, float x1, float y1, float z1, float e)
        : min_x(x0), min_y(y0), min_z(z0), max_x(x1), max_y(y1), max_z(z1), restitution(e) {}
    const char* name() const override { return "box_collider"; }
    void execute(FieldSet& fs, float) override {
        const float mn[3] = {min_x, min_y, min_z}, mx[3] = {max_x, max_y, max_z};
        check(fh_box_collider(fs.ctx.get(), fs.f("pos_x").data(), fs.f("pos_y").data(),
                              fs.f("pos_z").data(), fs.f("vel_x").data(), fs.f("vel_y").data(),
                              fs.f("vel_z").data(), (uint32_t)fs.particle_count, mn, mx,
                              restitution));
    }
};

// Modules run in order; a sph_fused followed by gravity / integrate / box is fused into one
// force pass with the same result (the build_pipeline fusion idea, manifest_runner.rs:334-379).
class Pipeline {
   public:
    void add(std::unique_ptr<SimModule> m) {
        modules_.push_back(std::move(m));
        fused_ = false;
    }
    size_t len() const { return modules_.size(); }
    void step_async(FieldSet& fs, float dt) {
        plan();
        for (SimModule* m : plan_) m->execute(fs, dt);
    }
    void step(FieldSet& fs, float dt) {
        step_async(fs, dt);
        fs.ctx.sync();
    }
    // `steps` substeps queued on the context stream.  When the (fused) plan is a single
    // SphFusedModule and `resident` is set, they are one fh_sph_fused_steps call: the state stays
    // in sorted order on the device and the fields are written after the last substep only
    // (nothing else reads them in between).
    void run_async(FieldSet& fs, float dt, size_t steps) {
        plan();
        if (resident && steps > 1 && plan_.size() == 1) {
            if (auto* sph = dynamic_cast<SphFusedModule*>(plan_[0])) {
                sph->execute_steps(fs, dt, (uint32_t)steps);
                return;
            }
        }
        for (size_t i = 0; i < steps; i++) step_async(fs, dt);
    }
    void run(FieldSet& fs, float dt, size_t steps) {  // modules/mod.rs:106-112
        run_async(fs, dt, steps);
        fs.ctx.sync();
    }
    // Record `substeps` substeps (run_async) into the context's graph (manifest_runner.rs:57-69)
    // and replay it (manifest_runner.rs:74-77).
    void capture(FieldSet& fs, float dt, size_t substeps) {
        plan();
        for (SimModule* m : plan_) m->prepare(fs);
        fs.ctx.sync();
        check(fh_graph_begin(fs.ctx.get()));
        try {
            run_async(fs, dt, substeps);
        } catch (...) {
            fh_graph_end(fs.ctx.get());
            throw;
        }
        check(fh_graph_end(fs.ctx.get()));
    }
    void replay(FieldSet& fs, uint32_t count) { check(fh_graph_launch(fs.ctx.get(), count)); }

    // run_manifest_streaming's loop (manifest_runner.rs:145-181): each step runs `substeps`
    // substeps; after step s with s % frame_interval == 0 (an interval of 0 counts as 1) the
    // binary frame (pack_frame) is copied to the host and passed to on_frame(frame_number,
    // bytes).  Returns the final positions (interleaved x y z), count, substeps run and elapsed
    // seconds, as SimResult does.
    struct StreamResult {
        std::vector<float> positions;
        size_t count = 0, steps = 0;
        double elapsed_secs = 0.0;
    };
    template <class OnFrame>
    StreamResult run_streaming(FieldSet& fs, float dt, size_t total_steps, size_t substeps,
                               size_t frame_interval, OnFrame on_frame);

    bool resident = true;

   private:
    void plan() {
        if (fused_) return;
        plan_.clear();
        fused_mods_.clear();
        for (size_t i = 0; i < modules_.size(); i++) {
            auto* sph = dynamic_cast<SphFusedModule*>(modules_[i].get());
            if (sph && !sph->has_epilogue) {
                auto f = std::make_unique<SphFusedModule>(*sph);
                size_t j = i + 1;
                if (j < modules_.size()) {
                    if (auto* g = dynamic_cast<GravityModule*>(modules_[j].get())) {
                        f->epilogue.flags |= FH_EPI_GRAVITY;
                        f->epilogue.gravity[0] = g->gx;
                        f->epilogue.gravity[1] = g->gy;
                        f->epilogue.gravity[2] = g->gz;
                        j++;
                    }
                }
                if (j < modules_.size() && dynamic_cast<IntegrateModule*>(modules_[j].get())) {
                    f->epilogue.flags |= FH_EPI_INTEGRATE;
                    j++;
                }
                if (j < modules_.size()) {
                    if (auto* b = dynamic_cast<BoxColliderModule*>(modules_[j].get())) {
                        f->epilogue.flags |= FH_EPI_BOX;
                        f->epilogue.box_min[0] = b->min_x;
                        f->epilogue.box_min[1] = b->min_y;
                        f->epilogue.box_min[2] = b->min_z;
                        f->epilogue.box_max[0] = b->max_x;
                        f->epilogue.box_max[1] = b->max_y;
                        f->epilogue.box_max[2] = b->max_z;
                        f->epilogue.restitution = b->restitution;
                        j++;
                    }
                }
                if (j > i + 1) {
                    f->has_epilogue = true;
                    plan_.push_back(f.get());
                    fused_mods_.push_back(std::move(f));
                    i = j - 1;
                    continue;
                }
            }
            plan_.push_back(modules_[i].get());
        }
        fused_ = true;
    }
    std::vector<std::unique_ptr<SimModule>> modules_;
    std::vector<std::unique_ptr<SimModule>> fused_mods_;
    std::vector<SimModule*> plan_;
    bool fused_ = false;
};

// The binary position frame of the streaming runner (FrameBuffer::set_frame, serve.rs:7-10,43-62):
// u32 frame number, u32 particle count n, then x y z per particle as f32, little-endian.
inline size_t frame_bytes(size_t n) { return 8 + 12 * n; }

// Packs the current positions of `fs` into `out` on the device (fh_pack_frame).  With
// device_counter (a device u32) the frame number is read from it and incremented there instead,
// so a captured graph emits consecutive frame numbers on its replays.
inline void pack_frame(FieldSet& fs, uint32_t frame, Array<uint8_t>& out,
                       uint32_t* device_counter = nullptr) {
    if (out.len() < frame_bytes(fs.particle_count))
        throw Error(FH_EINVAL, "frame buffer too small");
    check(fh_pack_frame(fs.ctx.get(), fs.f("pos_x").data(), fs.f("pos_y").data(),
                        fs.f("pos_z").data(), (uint32_t)fs.particle_count, frame, device_counter,
                        out.data()));
}

template <class OnFrame>
Pipeline::StreamResult Pipeline::run_streaming(FieldSet& fs, float dt, size_t total_steps,
                                               size_t substeps, size_t frame_interval,
                                               OnFrame on_frame) {
    const size_t interval = frame_interval ? frame_interval : 1;
    auto dev = Array<uint8_t>::zeros(frame_bytes(fs.particle_count));
    StreamResult r;
    const auto t0 = std::chrono::steady_clock::now();
    uint32_t frame_num = 0;
    for (size_t s = 0; s < total_steps; s++) {
        run_async(fs, dt, substeps);
        r.steps += substeps;
        if (s % interval == 0) {
            pack_frame(fs, frame_num, dev);
            fs.ctx.sync();
            const std::vector<uint8_t> host = dev.to_vec();
            on_frame(frame_num, host);
            frame_num++;
        }
    }
    fs.ctx.sync();
    r.elapsed_secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    pack_frame(fs, 0, dev);
    fs.ctx.sync();
    const std::vector<uint8_t> host = dev.to_vec();
    r.count = fs.particle_count;
    r.positions.resize(3 * fs.particle_count);
    for (size_t i = 0; i < r.positions.size(); i++) {
        uint32_t bits = (uint32_t)host[8 + 4 * i] | (uint32_t)host[9 + 4 * i] << 8 |
                        (uint32_t)host[10 + 4 * i] << 16 | (uint32_t)host[11 + 4 * i] << 24;
        float f;
        static_assert(sizeof f == sizeof bits, "f32");
        std::memcpy(&f, &bits, sizeof f);
        r.positions[i] = f;
    }
    return r;
}

}  // namespace forge
