"""Seeded synthetic inputs shared by the CPU and GPU tests.

Distributions follow the benchmark configurations: activations ~ N(0, 1),
weights ~ N(0, 0.02) in fp16, and the heavy-tailed W4A4 activations
(Student-t with 3 degrees of freedom, 1% of channels scaled by 20).
"""
import numpy as np


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def f16_bits(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def weights_f16(n: int, k: int, seed: int, std: float = 0.02) -> np.ndarray:
    return f16_bits(rng(seed).normal(0.0, std, size=(n, k)))


def normal_f32(m: int, k: int, seed: int) -> np.ndarray:
    return rng(seed).normal(0.0, 1.0, size=(m, k)).astype(np.float32)


def heavy_tailed(m: int, k: int, seed: int) -> np.ndarray:
    g = rng(seed)
    z = g.normal(size=(m, k))
    chi2 = (g.normal(size=(m, k)) ** 2 + g.normal(size=(m, k)) ** 2 + g.normal(size=(m, k)) ** 2)
    t = z / np.sqrt(chi2 / 3.0)
    outliers = g.choice(k, size=max(1, -(-k // 100)), replace=False)
    t[:, outliers] *= 20.0
    return t.astype(np.float32)


def rel_l2(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs_over_rms(a: np.ndarray, b: np.ndarray) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    rms = float(np.sqrt(np.mean(b * b)))
    return float(np.max(np.abs(a - b)) / max(rms, 1e-30))


# Output tolerance of the north star: rel-L2 <= 1e-3 and max-abs <= 2e-2 * rms(out).
REL_L2_TOL = 1e-3
MAX_ABS_RMS_TOL = 2e-2
