"""Deterministic synthetic inputs of the five benchmark configurations.

Every value is produced with integer arithmetic and IEEE float64 operations rounded once to
float32, so any IEEE host generates bit-identical buffers (their SHA-256 is recorded with each
result).  Random numbers: splitmix64 of a counter; stream s, element i uses counter
s * 2**40 + i; a uniform float is (u32 >> 8) * 2**-24, exactly representable in [0, 1).

Resolutions of the configuration text (BASELINE.json "configs"):
  c0  40 x 40 lattice columns in x, y at spacing 0.0125 and as many z-layers as 50,000 needs
      (31 full layers + 400), x fastest; points at the cell centres (i + 0.5) * spacing plus a
      jitter (2u - 1) * 1e-3 per coordinate.
  c1  16,777,216 points u^3 in [0,1)^3, key = floor(256x) + 256 floor(256y) + 65536 floor(256z),
      values 0..N-1, full 32-bit sort.
  c2  4,194,304 uniform points in [0,1)^3, r = cs = 0.0122 (float32), 82^3 cells.
  c3  128 x 128 lattice columns at spacing 0.005 with 64 z-layers (exactly 1,048,576), jitter
      (2u - 1) * 4e-4, h = cs = 0.01, 100^3 cells.
  c4  8,388,608 points: the first floor(0.9 N) from 64 isotropic Gaussians (particle i belongs to
      component i % 64; centres U[0,1)^3, sigma U[0.005, 0.05]; normal deviate = sum of 12
      uniforms - 6), the rest uniform; everything clamped into [0, 1).
SPH constants (c0, c3, c4): rho0 = 1000, k = 2000, mu = 0.01, restitution 0.3 (from
examples/dam-break.toml), particle mass = rho0 / N * 0.001 in float32 as
forge-manifest/src/manifest_runner.rs:367 computes it, gravity (0, -9.81, 0), dt = 1e-4, box
[0,1]^3.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import numpy as np

DEFAULT_SEED = 20261201
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, counters: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (counters.astype(np.uint64) + np.uint64(1)) * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def u32_stream(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    ctr = np.uint64(stream) * np.uint64(1 << 40) + np.arange(start, start + n, dtype=np.uint64)
    return (splitmix64(seed, ctr) >> np.uint64(32)).astype(np.uint32)


def uniform_f32(seed: int, stream: int, n: int, start: int = 0) -> np.ndarray:
    """Uniform floats in [0, 1): (u32 >> 8) * 2^-24, exact in float32."""
    m = u32_stream(seed, stream, n, start) >> np.uint32(8)
    return (m.astype(np.float64) * 2.0 ** -24).astype(np.float32)


def sha256(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def particle_mass(rest_density: float, n: int) -> float:
    """manifest_runner.rs:367: rest_density / n as f32 * 0.001, in float32."""
    return float(np.float32(np.float32(rest_density) / np.float32(n)) * np.float32(0.001))


@dataclass
class SphConfig:
    name: str
    n: int
    x: np.ndarray
    y: np.ndarray
    z: np.ndarray
    h: float
    cell_size: float
    dims: tuple
    mass: float
    gas_constant: float = 2000.0
    rest_density: float = 1000.0
    viscosity: float = 0.01
    gravity: tuple = (0.0, -9.81, 0.0)
    dt: float = 1e-4
    box_min: tuple = (0.0, 0.0, 0.0)
    box_max: tuple = (1.0, 1.0, 1.0)
    restitution: float = 0.3
    substeps: int = 1
    seed: int = DEFAULT_SEED
    extra: dict = field(default_factory=dict)

    @property
    def num_cells(self) -> int:
        return int(self.dims[0]) * int(self.dims[1]) * int(self.dims[2])

    def digest(self) -> str:
        return sha256(self.x, self.y, self.z)


def lattice(n: int, cols_x: int, cols_y: int, spacing: float, jitter: float, seed: int):
    i = np.arange(n, dtype=np.int64)
    ix, iy, iz = i % cols_x, (i // cols_x) % cols_y, i // (cols_x * cols_y)
    out = []
    for axis, idx in enumerate((ix, iy, iz)):
        u = uniform_f32(seed, axis, n).astype(np.float64)
        out.append(((idx + 0.5) * spacing + (2.0 * u - 1.0) * jitter).astype(np.float32))
    return out


def config0(seed: int = DEFAULT_SEED, n: int = 50_000) -> SphConfig:
    x, y, z = lattice(n, 40, 40, 0.0125, 1e-3, seed)
    return SphConfig("c0", n, x, y, z, h=0.025, cell_size=0.025, dims=(40, 40, 40),
                     mass=particle_mass(1000.0, n), substeps=10, seed=seed)


def config3(seed: int = DEFAULT_SEED, n: int = 1_048_576) -> SphConfig:
    x, y, z = lattice(n, 128, 128, 0.005, 4e-4, seed)
    return SphConfig("c3", n, x, y, z, h=0.01, cell_size=0.01, dims=(100, 100, 100),
                     mass=particle_mass(1000.0, n), substeps=1000, seed=seed)


def uniform_points(n: int, seed: int, first_stream: int = 0):
    return [uniform_f32(seed, first_stream + a, n) for a in range(3)]


def config1(seed: int = DEFAULT_SEED, n: int = 16_777_216):
    """Keys and values of the standalone sort (keys < 2^24, sorted on all 32 bits)."""
    m = [u32_stream(seed, a, n) >> np.uint32(8) for a in range(3)]  # 24-bit mantissas
    keys = (m[0] >> np.uint32(16)) + (m[1] >> np.uint32(16)) * np.uint32(256) + \
        (m[2] >> np.uint32(16)) * np.uint32(65536)
    vals = np.arange(n, dtype=np.uint32)
    return keys.astype(np.uint32), vals


def config2(seed: int = DEFAULT_SEED, n: int = 4_194_304):
    x, y, z = uniform_points(n, seed)
    r = float(np.float32(0.0122))
    return dict(name="c2", n=n, x=x, y=y, z=z, radius=r, cell_size=r, dims=(82, 82, 82),
                origin=(0.0, 0.0, 0.0), seed=seed)


def config4(seed: int = DEFAULT_SEED, n: int = 8_388_608, chunk: int = 1 << 20) -> SphConfig:
    n_g = (9 * n) // 10
    comps = 64
    centers = [uniform_f32(seed, 10 + a, comps).astype(np.float64) for a in range(3)]
    sigma = 0.005 + 0.045 * uniform_f32(seed, 13, comps).astype(np.float64)
    out = [np.empty(n, dtype=np.float32) for _ in range(3)]
    top = np.float32(1.0 - 2.0 ** -24)
    for start in range(0, n_g, chunk):
        m = min(chunk, n_g - start)
        k = np.arange(start, start + m) % comps
        for a in range(3):
            s = np.zeros(m, dtype=np.float64)
            for t in range(12):  # Irwin-Hall: 12 uniforms per deviate
                s += uniform_f32(seed, 20 + 12 * a + t, m, start)
            v = (centers[a][k] + sigma[k] * (s - 6.0)).astype(np.float32)
            out[a][start:start + m] = np.clip(v, np.float32(0.0), top)
    if n > n_g:
        for a in range(3):
            out[a][n_g:] = uniform_f32(seed, 60 + a, n - n_g, n_g)
    return SphConfig("c4", n, out[0], out[1], out[2], h=0.01, cell_size=0.01,
                     dims=(100, 100, 100), mass=particle_mass(1000.0, n), seed=seed)


def small_sph(n: int = 4096, seed: int = DEFAULT_SEED, cols: int = 16) -> SphConfig:
    """A reduced dam-break block for quick tests (c0 constants, lattice of `cols` columns)."""
    x, y, z = lattice(n, cols, cols, 0.0125, 1e-3, seed)
    return SphConfig("small", n, x, y, z, h=0.025, cell_size=0.025, dims=(40, 40, 40),
                     mass=particle_mass(1000.0, n), seed=seed)
