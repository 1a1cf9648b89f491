"""Seeded synthetic inputs for the benchmark configurations.

One generator produces the identical bytes for the CPU oracle and the GPU
upload.  Packed blocks follow the GGML layouts the reference decodes
(crates/bridge-quant-layout/src/k_quants.rs:7-20, iq2_s.rs:4-7, iq3_s.rs:4-7):

* Q4_K (144 B): d, dmin = f16(|N(0,1)| * 1e-2); eight random 6-bit (scale, min)
  pairs packed by inverting scale_min (k_quants.rs:231-240); uniform qs bytes.
* Q5_K (176 B): as Q4_K plus uniform qh bytes (5-bit quants).
* IQ2_S (82 B): d = f16(|N(0,1)| * 1e-3); uniform qs / signs / qh / scale bytes
  (so the 10-bit grid indices are uniform).
* IQ3_S (110 B): same construction (uniform 9-bit indices).
* activations: f32 N(0, 1).

numpy's PCG64 is deterministic for a given seed and numpy version.
"""
from __future__ import annotations

import numpy as np

F32, Q4_K, Q5_K, Q8_K, IQ3_S, IQ2_S = 0, 12, 13, 15, 21, 22
BLOCK_BYTES = {Q4_K: 144, Q5_K: 176, IQ2_S: 82, IQ3_S: 110}
TYPE_NAMES = {Q4_K: "Q4_K", Q5_K: "Q5_K", IQ2_S: "IQ2_S", IQ3_S: "IQ3_S", F32: "F32", Q8_K: "Q8_K"}


def _f16_abs_normal(rng: np.random.Generator, n: int, scale: float) -> np.ndarray:
    return (np.abs(rng.standard_normal(n)) * scale).astype(np.float16).view(np.uint16)


def pack_scale_min(scales: np.ndarray, mins: np.ndarray) -> np.ndarray:
    """Inverse of scale_min (k_quants.rs:231-240): [n, 8] 6-bit pairs -> [n, 12] bytes."""
    s = scales.astype(np.uint8) & 63
    m = mins.astype(np.uint8) & 63
    out = np.zeros((s.shape[0], 12), np.uint8)
    for j in range(4):
        out[:, j] = s[:, j] | ((s[:, j + 4] >> 4) << 6)
        out[:, j + 4] = m[:, j] | ((m[:, j + 4] >> 4) << 6)
        out[:, j + 8] = (s[:, j + 4] & 15) | ((m[:, j + 4] & 15) << 4)
    return out


def random_blocks(ty: int, n_blocks: int, rng: np.random.Generator) -> np.ndarray:
    """n_blocks packed blocks of type ty as a [n_blocks, block_bytes] uint8 array."""
    bb = BLOCK_BYTES[ty]
    blk = rng.integers(0, 256, size=(n_blocks, bb), dtype=np.uint8)
    if ty in (Q4_K, Q5_K):
        blk[:, 0:2] = _f16_abs_normal(rng, n_blocks, 1e-2).view(np.uint8).reshape(n_blocks, 2)
        blk[:, 2:4] = _f16_abs_normal(rng, n_blocks, 1e-2).view(np.uint8).reshape(n_blocks, 2)
        sc = rng.integers(0, 64, size=(n_blocks, 8))
        mn = rng.integers(0, 64, size=(n_blocks, 8))
        blk[:, 4:16] = pack_scale_min(sc, mn)
    else:
        blk[:, 0:2] = _f16_abs_normal(rng, n_blocks, 1e-3).view(np.uint8).reshape(n_blocks, 2)
    return blk


def random_matrix(ty: int, rows: int, k: int, seed: int) -> np.ndarray:
    """GGML [K, rows] packed matrix: rows x (K/256) blocks, row-major bytes."""
    assert k % 256 == 0
    rng = np.random.default_rng(seed)
    return random_blocks(ty, rows * (k // 256), rng).reshape(rows, -1)


def random_activations(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


def router_weights(n_experts: int, hidden: int, seed: int) -> np.ndarray:
    """F32 router [hidden, n_experts] GGML view, stored expert-major ([n_experts][hidden]), N(0, 0.02)."""
    return (np.random.default_rng(seed).standard_normal((n_experts, hidden)) * 0.02).astype(np.float32)


def zipf_routes(n_tokens: int, n_experts: int, top_k: int, s: float, seed: int) -> np.ndarray:
    """Per-token router logits with Zipf(s) expert popularity: Gumbel-top-k over
    log p_e, p_e proportional to rank^-s under a seeded random rank permutation."""
    rng = np.random.default_rng(seed)
    ranks = rng.permutation(n_experts) + 1
    logp = -s * np.log(ranks.astype(np.float64))
    g = rng.gumbel(size=(n_tokens, n_experts))
    return (logp[None, :] + g).astype(np.float32)
