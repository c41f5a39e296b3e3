"""Seeded synthetic inputs for the BASELINE configurations of the matvecQ8 path.

numpy's PCG64 generator (np.random.default_rng(seed)), standard normals by
its ziggurat: deterministic for a given numpy version and seed.  Inputs are
made once on the host and the same arrays go to the GPU and to any CPU
baseline (transcendental functions differ across engines, so nothing is
regenerated on the other side).

  cfg1  N=2048,  K=2048                 x ~ N(0,1), W ~ N(0, 0.02)
  cfg2  N=11008, K=4096                 (Llama-7B MLP up; the headline shape)
  cfg3  N=4096,  K=4099                 ragged K; 1% of rows carry one x50 outlier
  cfg4  decoder layer, hidden 2048, FFN 5632, 16 heads:
        q/k/v/o [2048,2048], gate/up [5632,2048], down [2048,5632]
  cfg5  N=151936, K=1024, M in {1,4,8,16} (vocab head, small-M batched)
"""
from __future__ import annotations

import numpy as np

CONFIGS = {
    "cfg1": {"N": 2048, "K": 2048, "seed": 1},
    "cfg2": {"N": 11008, "K": 4096, "seed": 2},
    "cfg3": {"N": 4096, "K": 4099, "seed": 3, "outlier_rows": 0.01, "outlier_scale": 50.0},
    "cfg5": {"N": 151936, "K": 1024, "seed": 5},
}

DECODER_LAYER = [  # cfg4: (name, N, K)
    ("wq", 2048, 2048), ("wk", 2048, 2048), ("wv", 2048, 2048), ("wo", 2048, 2048),
    ("wGate", 5632, 2048), ("wUp", 5632, 2048), ("wDown", 2048, 5632),
]
DECODER_SEED = 4
# prefill (matmulQ8): tokens in the prompt run through the cfg4 projections
PREFILL_TOKENS = 512


def weights_f32(rng: np.random.Generator, N: int, K: int, std: float = 0.02) -> np.ndarray:
    return (rng.standard_normal((N, K), dtype=np.float32) * np.float32(std)).reshape(-1)


def vectors_f32(rng: np.random.Generator, M: int, K: int) -> np.ndarray:
    return rng.standard_normal((M, K), dtype=np.float32).reshape(-1)


def make_config(name: str, M: int = 1):
    """Returns dict(N, K, M, w=f32 [N*K], x=f32 [M*K], outliers=row indices)."""
    c = CONFIGS[name]
    rng = np.random.default_rng(c["seed"])
    N, K = c["N"], c["K"]
    w = weights_f32(rng, N, K)
    outliers = np.array([], dtype=np.int64)
    if "outlier_rows" in c:
        count = int(round(N * c["outlier_rows"]))
        outliers = np.sort(rng.choice(N, size=count, replace=False))
        cols = rng.integers(0, K, size=count)
        w2 = w.reshape(N, K)
        w2[outliers, cols] *= np.float32(c["outlier_scale"])
    x = vectors_f32(rng, M, K)
    return {"N": N, "K": K, "M": M, "w": w, "x": x, "outliers": outliers}


def make_decoder_layer():
    rng = np.random.default_rng(DECODER_SEED)
    mats = [(name, N, K, weights_f32(rng, N, K)) for name, N, K in DECODER_LAYER]
    x_hidden = vectors_f32(rng, 1, 2048)
    x_ffn = vectors_f32(rng, 1, 5632)
    return mats, x_hidden, x_ffn


def matvec_bytes(N: int, K: int, M: int = 1) -> int:
    """Algorithmic HBM bytes of one matvecQ8 call: packed weight, scale, vectors in, outputs out."""
    W = (K + 3) // 4
    return N * W * 4 + 4 * N + 4 * K * M + 4 * N * M


def quantize_pack_bytes(N: int, K: int) -> int:
    W = (K + 3) // 4
    return 4 * N * K + N * W * 4 + 4 * N
