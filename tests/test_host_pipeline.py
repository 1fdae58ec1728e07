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
