"""Host-side pipeline construction (no GPU: modules are only built, never executed)."""
import numpy as np
import pytest


def test_build_pipeline_fuses_the_three_sph_forces(fh):
    """manifest_runner.rs:334-379: density + pressure + viscosity become one fused module,
    followed by the other forces, integrate and the constraints."""
    pipe = fh.build_pipeline([{"type": "sph_density", "smoothing_radius": 0.025},
                              {"type": "sph_pressure", "gas_constant": 2000.0,
                               "rest_density": 1000.0},
                              {"type": "sph_viscosity", "coefficient": 0.01},
                              {"type": "gravity", "value": [0, -9.81, 0]}],
                             [{"type": "box", "min": [0, 0, 0], "max": [1, 1, 1],
                               "restitution": 0.3}], n=50_000)
    assert [m.name() for m in pipe.modules] == ["sph_fused", "gravity", "integrate",
                                                "box_collider"]
    m = pipe.modules[0]
    assert m.cell_size == pytest.approx(0.05) and m.grid_dims == [32, 32, 32]


def test_build_pipeline_unfused_defaults(fh):
    """Without all three SPH forces build_pipeline does not fuse; pressure / viscosity take the
    reference's defaults (cell size 0.05, h from sph_density, masses of :452 and :478)."""
    pipe = fh.build_pipeline([{"type": "sph_density", "smoothing_radius": 0.02},
                              {"type": "sph_pressure", "gas_constant": 3000.0,
                               "rest_density": 500.0},
                              {"type": "gravity", "value": [0, -9.81, 0]}], [], n=1000)
    names = [m.name() for m in pipe.modules]
    assert names == ["sph_density", "sph_pressure", "gravity", "integrate"]
    d, p = pipe.modules[0], pipe.modules[1]
    assert d.cell_size == pytest.approx(0.04) and p.cell_size == pytest.approx(0.05)
    assert p.smoothing_radius == pytest.approx(0.02) and p.grid_dims == [32, 32, 32]
    assert p.particle_mass == pytest.approx(float(np.float32(500.0) / np.float32(1000) * np.float32(0.001)))


def test_build_pipeline_box_defaults_per_element(fh):
    """manifest_runner.rs:528-537: each missing min element is 0.0 and each missing max
    element 1.0 on its own; restitution 0.5 when absent (schema.rs:151-159)."""
    pipe = fh.build_pipeline([{"type": "gravity", "value": [0, -9.81, 0]}],
                             [{"type": "box", "min": [-0.5], "max": [2.0, 3.0]}], n=10)
    b = pipe.modules[-1]
    assert (b.min_x, b.min_y, b.min_z) == (-0.5, 0.0, 0.0)
    assert (b.max_x, b.max_y, b.max_z) == (2.0, 3.0, 1.0)
    assert b.restitution == 0.5
    # gravity: each missing element of `value` takes 0, -9.81, 0 (manifest_runner.rs:391-396)
    pipe = fh.build_pipeline([{"type": "gravity", "value": [1.5]}], [], n=10)
    g = pipe.modules[0]
    assert (g.gx, g.gy, g.gz) == (1.5, pytest.approx(-9.81), 0.0)


def test_init_fields_names_and_defaults(fh):
    """init_fields (manifest_runner.rs:192-233): vec3f fields split into _x/_y/_z with position
    -> pos and velocity -> vel; f32 fields keep their name; missing vel / pos are zeros."""
    out = fh.init_field_arrays([{"name": "position", "type": "vec3f",
                                 "init": {"type": "constant", "value": [0.25, -1.0]}},
                                {"name": "temperature", "type": "f32",
                                 "init": {"type": "constant", "value": [300.0]}},
                                {"name": "mass", "type": "f32"}], n=5)
    assert sorted(out) == ["mass", "pos_x", "pos_y", "pos_z", "temperature", "vel_x", "vel_y",
                           "vel_z"]
    assert np.all(out["pos_x"] == np.float32(0.25)) and np.all(out["pos_y"] == -1.0)
    assert np.all(out["pos_z"] == 0.0)  # a missing element of `value` is 0
    assert np.all(out["temperature"] == 300.0) and np.all(out["mass"] == 0.0)
    for k in ("vel_x", "vel_y", "vel_z"):
        assert out[k].dtype == np.float32 and np.all(out[k] == 0.0)
    # no position field at all: pos_* are zeros; "vel" is the base name of "velocity"
    out = fh.init_field_arrays([{"name": "velocity", "init": {"type": "constant",
                                                              "value": [1, 2, 3]}}], n=3)
    assert out["vel_z"].tolist() == [3.0] * 3 and out["pos_x"].tolist() == [0.0] * 3


def test_init_fields_grid_closed_form(fh):
    """init_vec3 Grid (manifest_runner.rs:281-295): side = ceil(sqrt(n)), particle i at
    (ox + (i % side) sp, oy, oz + (i // side) sp) in float32."""
    n, sp, o = 10, 0.125, (1.0, 2.0, -3.0)
    out = fh.init_field_arrays([{"name": "pos", "init": {"type": "grid", "spacing": sp,
                                                         "origin": list(o)}}], n=n)
    side = 4  # ceil(sqrt(10))
    for i in range(n):
        assert out["pos_x"][i] == np.float32(o[0] + (i % side) * sp)  # exact: sp is 2^-3
        assert out["pos_y"][i] == np.float32(o[1])
        assert out["pos_z"][i] == np.float32(o[2] + (i // side) * sp)
    # spacing / origin defaults 0.1 and 0 (schema.rs:85-86), origin elements one by one
    out = fh.init_field_arrays([{"name": "pos", "init": {"type": "grid", "origin": [0.5]}}], n=4)
    assert out["pos_x"].tolist() == [np.float32(0.5), np.float32(0.5) + np.float32(0.1)] * 2
    assert out["pos_z"].tolist() == [0.0, 0.0, np.float32(0.1), np.float32(0.1)]


def test_init_fields_random_range(fh):
    """init_vec3 Random (manifest_runner.rs:257-268): uniform in [min, max) per component, each
    missing element -1 / 1; seeded here, so two calls agree (the reference's is unseeded)."""
    defs = [{"name": "position", "init": {"type": "random", "min": [0.0, 0.0, 0.0],
                                          "max": [1.0, 2.0, 0.5]}},
            {"name": "velocity", "init": {"type": "random", "min": [0.25]}}]
    a = fh.init_field_arrays(defs, n=20_000, seed=3)
    b = fh.init_field_arrays(defs, n=20_000, seed=3)
    for k in a:
        assert np.array_equal(a[k], b[k])
    for k, lo, hi in (("pos_x", 0, 1), ("pos_y", 0, 2), ("pos_z", 0, 0.5), ("vel_x", 0.25, 1),
                      ("vel_y", -1, 1), ("vel_z", -1, 1)):
        v = a[k]
        assert v.min() >= lo and v.max() < hi, k
        assert v.max() - v.min() > 0.99 * (hi - lo), k  # spread over the whole range
    assert not np.array_equal(a["pos_x"], a["pos_y"])  # independent streams
