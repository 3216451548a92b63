"""The reference's seeded correctness cases, restated -- TEST INFRASTRUCTURE ONLY.

MHA   tests/fused/cases.py:27-86      84 cases; Q, K ~ N(0,1)*sigma, V ~ N(0,1), fp16
GQA   tests/gqa/cases_gqa.py:28-97    96 cases; K/V drawn at H_kv heads (never pre-expanded)
bwd   tests/backward/cases_backward.py:20-79   7 shapes (B, H, N, D, sigma)

Inputs come from numpy.random.default_rng(zlib.crc32(case.id)), drawn in the
order Q, K, V with standard_normal(shape, dtype=float32), scaled, then cast -- the
reference's exact recipe, so the fp16 inputs match it bit for bit on the same
numpy version.  The reference draws its backward inputs from a CUDA torch
generator, which cannot be reproduced off-GPU; the backward cases here draw
from numpy.random.default_rng(N + D) instead (same shapes, same seed value).
"""

import zlib
from dataclasses import dataclass

import numpy as np

HEAD_DIMS = (32, 64, 128)
SEQ_LENS = (128, 512, 2048, 8192)
BATCH_HEADS = ((1, 1), (2, 8), (3, 5))
MAX_BATCH_HEADS = (16, 32)
MAX_SHAPE_SEQ_LENS = (128, 512)
MAGNITUDES = {"tiny": 0.03, "large": 7.0}

GQA_BATCH = 4
GQA_NUM_Q_HEADS = 8
GQA_NUM_KV_HEADS = (1, 2, 4, 8)

BWD_CASE_SHAPES = (
    (1, 1, 128, 64, 1.0),
    (2, 4, 256, 64, 1.0),
    (2, 4, 512, 128, 1.0),
    (1, 2, 1024, 64, 3.0),
    (2, 8, 2048, 64, 1.0),
    (2, 8, 2048, 128, 1.0),
    (1, 4, 512, 64, 7.0),
)


@dataclass(frozen=True)
class Case:
    """One MHA case (tests/fused/cases.py:27-53)."""
    B: int
    H: int
    N: int
    D: int
    magnitude: str

    @property
    def id(self) -> str:
        return f"B{self.B}_H{self.H}_N{self.N}_D{self.D}_{self.magnitude}"

    @property
    def sigma(self) -> float:
        return MAGNITUDES[self.magnitude]

    @property
    def seed(self) -> int:
        return zlib.crc32(self.id.encode())


def all_cases():
    """The 84 MHA cases in the reference's order (tests/fused/cases.py:56-72)."""
    cases = [Case(B, H, N, D, mag)
             for D in HEAD_DIMS for N in SEQ_LENS for mag in MAGNITUDES for B, H in BATCH_HEADS]
    B, H = MAX_BATCH_HEADS
    cases += [Case(B, H, N, D, mag)
              for N in MAX_SHAPE_SEQ_LENS for D in HEAD_DIMS for mag in MAGNITUDES]
    return cases


def make_inputs(case, dtype=np.float16):
    """Q, K, V float16 arrays [B, H, N, D] (tests/fused/cases.py:75-86).

    dtype=np.float32 returns the values before the fp16 cast (for a bf16 cast done in torch)."""
    rng = np.random.default_rng(case.seed)
    shape = (case.B, case.H, case.N, case.D)
    q = rng.standard_normal(shape, dtype=np.float32) * case.sigma
    k = rng.standard_normal(shape, dtype=np.float32) * case.sigma
    v = rng.standard_normal(shape, dtype=np.float32)
    return q.astype(dtype), k.astype(dtype), v.astype(dtype)


@dataclass(frozen=True)
class GqaCase:
    """One GQA case (tests/gqa/cases_gqa.py:37-63)."""
    B: int
    H: int
    H_kv: int
    N: int
    D: int
    magnitude: str

    def __post_init__(self):
        if self.H % self.H_kv != 0:
            raise ValueError(f"H_kv={self.H_kv} must divide H={self.H}")

    @property
    def group(self) -> int:
        return self.H // self.H_kv

    @property
    def id(self) -> str:
        return f"B{self.B}_H{self.H}_Hkv{self.H_kv}_N{self.N}_D{self.D}_{self.magnitude}"

    @property
    def sigma(self) -> float:
        return MAGNITUDES[self.magnitude]

    @property
    def seed(self) -> int:
        return zlib.crc32(self.id.encode())


def all_gqa_cases():
    """The 96 GQA cases in the reference's order (tests/gqa/cases_gqa.py:66-74)."""
    return [GqaCase(GQA_BATCH, GQA_NUM_Q_HEADS, H_kv, N, D, mag)
            for D in HEAD_DIMS for N in SEQ_LENS for mag in MAGNITUDES for H_kv in GQA_NUM_KV_HEADS]


def make_gqa_inputs(case, dtype=np.float16):
    """Q [B, H, N, D], K and V [B, H_kv, N, D] (tests/gqa/cases_gqa.py:77-90)."""
    rng = np.random.default_rng(case.seed)
    q_shape = (case.B, case.H, case.N, case.D)
    kv_shape = (case.B, case.H_kv, case.N, case.D)
    q = rng.standard_normal(q_shape, dtype=np.float32) * case.sigma
    k = rng.standard_normal(kv_shape, dtype=np.float32) * case.sigma
    v = rng.standard_normal(kv_shape, dtype=np.float32)
    return q.astype(dtype), k.astype(dtype), v.astype(dtype)


@dataclass(frozen=True)
class BwdCase:
    """One backward case (tests/backward/cases_backward.py:37-56)."""
    B: int
    H: int
    N: int
    D: int
    sigma: float

    @property
    def id(self) -> str:
        return f"B{self.B}_H{self.H}_N{self.N}_D{self.D}_s{self.sigma:g}"

    @property
    def seed(self) -> int:
        return self.N + self.D


def all_bwd_cases():
    return [BwdCase(*s) for s in BWD_CASE_SHAPES]


def make_bwd_inputs(case, dtype=np.float16):
    """q, k, v ~ N(0,1)*sigma and dO ~ N(0,1), drawn in that order from default_rng(N + D)."""
    rng = np.random.default_rng(case.seed)
    shape = (case.B, case.H, case.N, case.D)
    q, k, v = (rng.standard_normal(shape, dtype=np.float32) * case.sigma for _ in range(3))
    do = rng.standard_normal(shape, dtype=np.float32)
    return q.astype(dtype), k.astype(dtype), v.astype(dtype), do.astype(dtype)


def normal_inputs(shapes, seed, scale=1.0):
    """Arrays ~ N(0,1)*scale in float32 from default_rng(seed), drawn in the given order.

    Used for the full-size workloads (MHA B4 H32 S4096 D128, GQA, MQA, backward)."""
    rng = np.random.default_rng(seed)
    return [rng.standard_normal(s, dtype=np.float32) * np.float32(scale) for s in shapes]
