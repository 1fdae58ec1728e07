// test_mirror.cpp -- the reference's own hash-grid / radix-sort tests and one SPH pipeline
// step, written against the C++ host mirror (include/forge_hip.hpp) and run on the GPU.
//   tests/radix_sort_test.rs:14-48    test_radix_sort_small
//   tests/radix_sort_test.rs:94-137   test_radix_sort_compare_cpu_reference (with stability)
//   tests/radix_sort_test.rs:139-171  test_find_cell_boundaries
//   tests/hashgrid_test.rs:6-36       test_hashgrid_basic
//   tests/hashgrid_test.rs:38-88      test_hashgrid_uniform_distribution (exactly 8)
// plus a dam-break Pipeline step checked against the CPU oracle (oracle/oracle.h), a graph
// replay checked against eager steps, resident substeps against per-substep ones, the CSR cell
// ranges of sorted keys, the standalone force pass against the oracle, and the binary frames of
// the streaming runner.  Prints one line per test; exit status 0 iff all pass.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <vector>

#include "../../include/forge_hip.hpp"
#include "../../oracle/oracle.h"

using forge::Array;

static int failures = 0;
#define EXPECT(cond, msg)                                              \
    do {                                                               \
        if (!(cond)) {                                                 \
            std::printf("FAIL %s: %s (line %d)\n", __func__, msg, __LINE__); \
            failures++;                                                \
            return;                                                    \
        }                                                              \
    } while (0)

static std::vector<uint32_t> xorshift(uint32_t s, size_t n, uint32_t mask) {
    std::vector<uint32_t> v(n);
    for (auto& x : v) {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        x = s & mask;
    }
    return v;
}

static void test_radix_sort_small(forge::Context& ctx) {
    std::vector<uint32_t> kd = {15, 3, 7, 1, 9, 0, 12, 5, 8, 2, 14, 6, 11, 4, 13, 10};
    std::vector<uint32_t> vd(16);
    std::iota(vd.begin(), vd.end(), 0u);
    auto keys = Array<uint32_t>::from_vec(kd);
    auto vals = Array<uint32_t>::from_vec(vd);
    forge::RadixSorter sorter(ctx, 16);
    sorter.sort(keys, vals, 16, 4);
    ctx.sync();
    auto k = keys.to_vec(), v = vals.to_vec();
    for (uint32_t i = 0; i < 16; i++) EXPECT(k[i] == i, "keys not sorted");
    const uint32_t exp[16] = {5, 3, 9, 1, 13, 7, 11, 2, 8, 4, 15, 12, 6, 14, 10, 0};
    for (int i = 0; i < 16; i++) EXPECT(v[i] == exp[i], "key-value mismatch");
    std::printf("PASS test_radix_sort_small\n");
}

static void test_radix_sort_compare_cpu_reference(forge::Context& ctx) {
    const size_t n = 5000;
    auto kd = xorshift(42, n, 0xFFFF);
    std::vector<uint32_t> vd(n);
    std::iota(vd.begin(), vd.end(), 0u);
    std::vector<std::pair<uint32_t, uint32_t>> cpu(n);
    for (size_t i = 0; i < n; i++) cpu[i] = {kd[i], vd[i]};
    std::stable_sort(cpu.begin(), cpu.end(),
                     [](const auto& a, const auto& b) { return a.first < b.first; });
    auto keys = Array<uint32_t>::from_vec(kd);
    auto vals = Array<uint32_t>::from_vec(vd);
    forge::RadixSorter(ctx, n).sort(keys, vals, n, 16);
    ctx.sync();
    auto k = keys.to_vec(), v = vals.to_vec();
    for (size_t i = 0; i < n; i++) {
        EXPECT(k[i] == cpu[i].first, "keys differ from the CPU stable sort");
        EXPECT(v[i] == cpu[i].second, "values differ from the CPU stable sort (stability)");
    }
    std::printf("PASS test_radix_sort_compare_cpu_reference\n");
}

static void test_find_cell_boundaries(forge::Context& ctx) {
    auto ids = Array<uint32_t>::from_vec({0, 0, 1, 1, 1, 3, 3, 5});
    auto cs = Array<uint32_t>::zeros(8), ce = Array<uint32_t>::zeros(8);
    forge::find_cell_boundaries(ctx, ids, cs, ce, 8, 8);
    ctx.sync();
    auto s = cs.to_vec(), e = ce.to_vec();
    EXPECT(s[0] == 0 && e[0] == 2, "cell 0");
    EXPECT(s[1] == 2 && e[1] == 5, "cell 1");
    EXPECT(s[3] == 5 && e[3] == 7, "cell 3");
    EXPECT(s[5] == 7 && e[5] == 8, "cell 5");
    EXPECT(s[2] == 0xFFFFFFFFu && e[2] == 0, "empty cell 2 sentinel");
    std::printf("PASS test_find_cell_boundaries\n");
}

static void test_hashgrid_basic(forge::Context& ctx) {
    forge::HashGrid grid(ctx, 1.0f, 10, 10, 10, {0, 0, 0}, 100);
    std::vector<forge::Vec3f> pos = {{5.0f, 5.0f, 5.0f}, {5.1f, 5.0f, 5.0f}, {5.5f, 5.5f, 5.5f},
                                     {9.0f, 9.0f, 9.0f}};
    auto p = Array<forge::Vec3f>::from_vec(pos);
    grid.build(p);
    auto nb = grid.query_neighbors(pos[0], 1.0f, p);
    auto has = [&](uint32_t i) { return std::find(nb.begin(), nb.end(), i) != nb.end(); };
    EXPECT(has(0) && has(1) && has(2), "should find 0, 1, 2");
    EXPECT(!has(3), "should not find 3");
    std::printf("PASS test_hashgrid_basic\n");
}

static void test_hashgrid_uniform_distribution(forge::Context& ctx) {
    forge::HashGrid grid(ctx, 2.0f, 5, 5, 5, {0, 0, 0}, 1000);
    std::vector<forge::Vec3f> pos(1000);
    for (int i = 0; i < 1000; i++)
        pos[i] = {(float)(i % 10) + 0.5f, (float)((i / 10) % 10) + 0.5f, (float)(i / 100) + 0.5f};
    auto p = Array<forge::Vec3f>::from_vec(pos);
    grid.build(p);
    forge::Vec3f c = {5.0f, 5.0f, 5.0f};
    auto nb = grid.query_neighbors(c, 1.5f, p);
    EXPECT(nb.size() == 8, "the 2x2x2 block around the centre");
    for (uint32_t i : nb) {
        float dx = pos[i].x - c.x, dy = pos[i].y - c.y, dz = pos[i].z - c.z;
        EXPECT(std::sqrt(dx * dx + dy * dy + dz * dz) <= 1.5f, "neighbour beyond radius");
    }
    std::printf("PASS test_hashgrid_uniform_distribution\n");
}

static void dam_break(size_t n, std::vector<float>* st) {
    for (int a = 0; a < 6; a++) st[a].assign(n, 0.0f);
    for (size_t i = 0; i < n; i++) {  // 16 x 16 columns, spacing 0.0125, deterministic offsets
        st[0][i] = (float)((i % 16) + 0.5) * 0.0125f + 1e-4f * (float)(i % 7);
        st[1][i] = (float)((i / 16 % 16) + 0.5) * 0.0125f + 1e-4f * (float)(i % 5);
        st[2][i] = (float)((i / 256) + 0.5) * 0.0125f + 1e-4f * (float)(i % 3);
    }
}

static void test_pipeline_step_matches_oracle(forge::Context& ctx) {
    const size_t n = 4096;
    const float h = 0.025f, m = 1000.0f / (float)n * 0.001f, dt = 1e-4f;
    std::vector<float> st[6];
    dam_break(n, st);
    forge::FieldSet fs(ctx, n);
    const char* names[6] = {"pos_x", "pos_y", "pos_z", "vel_x", "vel_y", "vel_z"};
    for (int a = 0; a < 6; a++) fs.add_f32(names[a], st[a]);
    forge::Pipeline pipe;
    pipe.add(std::make_unique<forge::SphFusedModule>(h, h, 40, 40, 40, m, 2000.0f, 1000.0f, 0.01f));
    pipe.add(std::make_unique<forge::GravityModule>(0.0f, -9.81f, 0.0f));
    pipe.add(std::make_unique<forge::IntegrateModule>());
    pipe.add(std::make_unique<forge::BoxColliderModule>(0, 0, 0, 1, 1, 1, 0.3f));
    pipe.step(fs, dt);
    or_sph_params p{h, h, {40, 40, 40}, m, 2000.0f, 1000.0f, 0.01f};
    const float g[3] = {0, -9.81f, 0}, mn[3] = {0, 0, 0}, mx[3] = {1, 1, 1};
    std::vector<float> rho(n), acc(3 * n);
    or_sph_step(&p, 7, g, mn, mx, 0.3f, st[0].data(), st[1].data(), st[2].data(), st[3].data(),
                st[4].data(), st[5].data(), (uint32_t)n, dt, rho.data(), acc.data());
    auto grho = fs.f("density").to_vec();
    for (size_t i = 0; i < n; i++)
        EXPECT(std::fabs(grho[i] - rho[i]) <= 1e-4f * std::fabs(rho[i]), "density vs oracle");
    std::printf("PASS test_pipeline_step_matches_oracle\n");
}

static void test_graph_replay_matches_eager(forge::Context& ctx) {
    const size_t n = 4096;
    const float h = 0.025f, m = 1000.0f / (float)n * 0.001f, dt = 1e-4f;
    std::vector<float> st[6];
    dam_break(n, st);
    const char* names[6] = {"pos_x", "pos_y", "pos_z", "vel_x", "vel_y", "vel_z"};
    forge::FieldSet a(ctx, n), b(ctx, n);
    for (int q = 0; q < 6; q++) {
        a.add_f32(names[q], st[q]);
        b.add_f32(names[q], st[q]);
    }
    auto build = [&](forge::Pipeline& p) {
        p.add(std::make_unique<forge::SphFusedModule>(h, h, 40, 40, 40, m, 2000.0f, 1000.0f, 0.01f));
        p.add(std::make_unique<forge::GravityModule>(0.0f, -9.81f, 0.0f));
        p.add(std::make_unique<forge::IntegrateModule>());
        p.add(std::make_unique<forge::BoxColliderModule>(0, 0, 0, 1, 1, 1, 0.3f));
    };
    forge::Pipeline pe, pg;
    build(pe);
    build(pg);
    pg.capture(b, dt, 5);
    for (int rep = 0; rep < 2; rep++) {
        pe.run(a, dt, 5);
        pg.replay(b, 1);
        ctx.sync();
        for (int q = 0; q < 6; q++) {
            auto x = a.f(names[q]).to_vec(), y = b.f(names[q]).to_vec();
            EXPECT(x == y, "graph replay differs from eager steps");
        }
    }
    std::printf("PASS test_graph_replay_matches_eager\n");
}

static void test_cell_start_csr(forge::Context& ctx) {
    // sorted keys, one of them (9) outside the 8-cell grid
    std::vector<uint32_t> kd = {0, 0, 1, 1, 1, 3, 3, 5, 9};
    auto keys = Array<uint32_t>::from_vec(kd);
    auto cs = Array<uint32_t>::zeros(9);
    forge::cell_start_csr(ctx, keys, kd.size(), 8, cs);
    ctx.sync();
    std::vector<uint32_t> exp(9);
    or_cell_start_csr(kd.data(), (uint32_t)kd.size(), 8, exp.data());
    const std::vector<uint32_t> lit = {0, 2, 5, 5, 7, 7, 8, 8, 8};
    EXPECT(exp == lit, "oracle: number of keys below each cell");
    EXPECT(cs.to_vec() == lit, "cell_start from sorted keys");
    std::printf("PASS test_cell_start_csr\n");
}

static void fill(forge::FieldSet& fs, std::vector<float>* st) {
    const char* names[6] = {"pos_x", "pos_y", "pos_z", "vel_x", "vel_y", "vel_z"};
    for (int a = 0; a < 6; a++) fs.add_f32(names[a], st[a]);
}

static void dam_break_pipeline(forge::Pipeline& p, float h, float m) {
    p.add(std::make_unique<forge::SphFusedModule>(h, h, 40, 40, 40, m, 2000.0f, 1000.0f, 0.01f));
    p.add(std::make_unique<forge::GravityModule>(0.0f, -9.81f, 0.0f));
    p.add(std::make_unique<forge::IntegrateModule>());
    p.add(std::make_unique<forge::BoxColliderModule>(0, 0, 0, 1, 1, 1, 0.3f));
}

// Pipeline::run keeps the state resident (one fh_sph_fused_steps call); the substeps then visit a
// cell's particles in the previous substep's order, so results match the per-substep form up to
// rounding.
static void test_resident_run_matches_substeps(forge::Context& ctx) {
    const size_t n = 4096;
    const float h = 0.025f, m = 1000.0f / (float)n * 0.001f, dt = 1e-4f;
    std::vector<float> st[6];
    dam_break(n, st);
    forge::FieldSet a(ctx, n), b(ctx, n);
    fill(a, st);
    fill(b, st);
    forge::Pipeline pr, ps;
    dam_break_pipeline(pr, h, m);
    dam_break_pipeline(ps, h, m);
    ps.resident = false;
    pr.run(a, dt, 3);
    ps.run(b, dt, 3);
    auto ra = a.f("density").to_vec(), rb = b.f("density").to_vec();
    for (size_t i = 0; i < n; i++)
        EXPECT(std::fabs(ra[i] - rb[i]) <= 1e-4f * std::fabs(rb[i]), "density");
    const char* names[3] = {"pos_x", "pos_y", "pos_z"};
    for (int q = 0; q < 3; q++) {
        auto x = a.f(names[q]).to_vec(), y = b.f(names[q]).to_vec();
        for (size_t i = 0; i < n; i++)
            EXPECT(std::fabs(x[i] - y[i]) <= 1e-6f + 1e-5f * std::fabs(y[i]), "position");
    }
    std::printf("PASS test_resident_run_matches_substeps\n");
}

// SphFusedModule::execute_force over the grid and densities SphDensityModule left in the field
// set equals the oracle's fused pass on the same inputs bit for bit (the caller's grid is walked
// with the reference's expressions and neighbour order).
static void test_force_after_density_matches_oracle(forge::Context& ctx) {
    const size_t n = 4096;
    const float h = 0.025f, m = 1000.0f / (float)n * 0.001f, dt = 1e-4f;
    std::vector<float> st[6];
    dam_break(n, st);
    for (size_t i = 0; i < n; i++) {  // velocities, so the viscosity term is not zero
        st[3][i] = 0.1f * (float)(i % 11) - 0.5f;
        st[4][i] = 0.05f * (float)(i % 7);
        st[5][i] = -0.02f * (float)(i % 5);
    }
    forge::FieldSet fs(ctx, n);
    fill(fs, st);
    forge::SphDensityModule dens(h, h, 40, 40, 40, m);
    forge::SphFusedModule sph(h, h, 40, 40, 40, m, 2000.0f, 1000.0f, 0.01f);
    dens.execute(fs, dt);
    auto acc = Array<float>::zeros(3 * n);
    sph.execute_force(fs, dt, acc.data());
    ctx.sync();
    auto rho = fs.f("density").to_vec();
    auto cs = fs.u("cell_start").to_vec(), si = fs.u("sorted_indices").to_vec();
    or_sph_params p{h, h, {40, 40, 40}, m, 2000.0f, 1000.0f, 0.01f};
    std::vector<float> vout(3 * n), aout(3 * n);
    or_sph_force(&p, st[0].data(), st[1].data(), st[2].data(), st[3].data(), st[4].data(),
                 st[5].data(), rho.data(), (uint32_t)n, cs.data(), si.data(), dt, vout.data(),
                 aout.data());
    auto ga = acc.to_vec();
    const char* names[3] = {"vel_x", "vel_y", "vel_z"};
    for (int q = 0; q < 3; q++) {
        auto v = fs.f(names[q]).to_vec();
        for (size_t i = 0; i < n; i++) {
            EXPECT(v[i] == vout[(size_t)q * n + i], "velocity vs oracle");
            EXPECT(ga[(size_t)q * n + i] == aout[(size_t)q * n + i], "acceleration vs oracle");
        }
    }
    std::printf("PASS test_force_after_density_matches_oracle\n");
}

static std::vector<float> frame_floats(const std::vector<uint8_t>& f, uint32_t* frame,
                                       uint32_t* count) {
    auto u32 = [&](size_t o) {
        return (uint32_t)f[o] | (uint32_t)f[o + 1] << 8 | (uint32_t)f[o + 2] << 16 |
               (uint32_t)f[o + 3] << 24;
    };
    *frame = u32(0);
    *count = u32(4);
    std::vector<float> x((f.size() - 8) / 4);
    for (size_t i = 0; i < x.size(); i++) {
        const uint32_t b = u32(8 + 4 * i);
        std::memcpy(&x[i], &b, 4);
    }
    return x;
}

static void test_pack_frame_and_streaming(forge::Context& ctx) {
    const size_t n = 4096;
    const float h = 0.025f, m = 1000.0f / (float)n * 0.001f, dt = 1e-4f;
    std::vector<float> st[6];
    dam_break(n, st);
    forge::FieldSet fs(ctx, n);
    fill(fs, st);
    auto out = Array<uint8_t>::zeros(forge::frame_bytes(n));
    forge::pack_frame(fs, 7, out);
    ctx.sync();
    uint32_t frame = 0, count = 0;
    auto x = frame_floats(out.to_vec(), &frame, &count);
    EXPECT(frame == 7 && count == n, "frame header");
    for (size_t i = 0; i < n; i++)
        for (int q = 0; q < 3; q++) EXPECT(x[3 * i + q] == st[q][i], "interleaved positions");
    forge::Pipeline p;
    dam_break_pipeline(p, h, m);
    std::vector<uint32_t> seen;
    std::vector<float> last;
    auto r = p.run_streaming(fs, dt, 5, 2, 2, [&](uint32_t f, const std::vector<uint8_t>& bytes) {
        uint32_t fr = 0, c = 0;
        last = frame_floats(bytes, &fr, &c);
        EXPECT(fr == f && c == n, "streamed frame header");
        seen.push_back(f);
    });
    EXPECT(seen == std::vector<uint32_t>({0, 1, 2}), "frames after steps 0, 2 and 4");
    EXPECT(r.steps == 10 && r.count == n, "substeps run");
    EXPECT(r.positions == last, "final positions equal the last frame (step 4 is the last)");
    auto px = fs.f("pos_x").to_vec();
    for (size_t i = 0; i < n; i++) EXPECT(r.positions[3 * i] == px[i], "final positions");
    std::printf("PASS test_pack_frame_and_streaming\n");
}

int main() {
    try {
        forge::Context ctx(1 << 16, 1 << 16);
        test_radix_sort_small(ctx);
        test_radix_sort_compare_cpu_reference(ctx);
        test_find_cell_boundaries(ctx);
        test_hashgrid_basic(ctx);
        test_hashgrid_uniform_distribution(ctx);
        test_pipeline_step_matches_oracle(ctx);
        test_graph_replay_matches_eager(ctx);
        test_cell_start_csr(ctx);
        test_resident_run_matches_substeps(ctx);
        test_force_after_density_matches_oracle(ctx);
        test_pack_frame_and_streaming(ctx);
    } catch (const forge::Error& e) {
        std::printf("FAIL exception %d: %s\n", e.code(), e.what());
        return 2;
    }
    std::printf("%s (%d failures)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
