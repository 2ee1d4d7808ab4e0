"""Seeded synthetic inputs of the benchmark shapes (mirrors the role of the
reference's shared case definitions, python/sglang/benchmark/remnant/cases.py).

Latents: BF16 N(0,1) * sigma_c, sigma_c log-uniform on [0.1, 10] per
coordinate (shared across records), seed 20260919 (the reference protocol
seed, decode-store manifest.json). RoPE table: torch.polar(1, pos * theta_j)
with theta_j = 10000^(-j/32) evaluated in float32.
"""

from __future__ import annotations

import math

import numpy as np
import torch

SEED = 20260919
HEAD_DIM = 512


def latents(rows: int, seed: int = SEED, dtype=torch.bfloat16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    sigma = torch.exp(torch.empty(HEAD_DIM).uniform_(math.log(0.1), math.log(10.0), generator=g))
    x = torch.randn(rows, HEAD_DIM, generator=g) * sigma
    return x.to(dtype)


def rope_inv_freq() -> torch.Tensor:
    """float32 [32]: theta_j = 10000^(-j/32), the inverse frequencies of the table."""
    return 1.0 / (10000.0 ** (torch.arange(0, 64, 2, dtype=torch.float32) / 64))


def rope_freqs(positions: int) -> torch.Tensor:
    """complex64 [positions, 32]: polar(1, pos * theta_j) with the angle in float32."""
    ang = torch.outer(torch.arange(positions, dtype=torch.float32), rope_inv_freq())
    return torch.polar(torch.ones_like(ang), ang)


def paged_requests(context_records, seed: int, pool_pages: int | None = None):
    """Random paged block tables for requests of the given record counts.
    Returns (block_table int32 [B, max_blocks] padded with -1, pool_pages)."""
    rng = np.random.default_rng(seed)
    blocks = [math.ceil(c / 64) for c in context_records]
    total = sum(blocks)
    pages = pool_pages if pool_pages is not None else total
    perm = rng.permutation(pages)[:total]
    width = max(blocks) if blocks else 0
    table = np.full((len(blocks), width), -1, np.int32)
    at = 0
    for b, n in enumerate(blocks):
        table[b, :n] = perm[at:at + n]
        at += n
    return table, pages


def topk_indices(context_records, q_len: int, topk: int, seed: int):
    """Uniform top-k without replacement per token; -1 pads short contexts.
    Returns (indices int32 [B, q_len, topk], lengths int32 [B*q_len])."""
    rng = np.random.default_rng(seed)
    idx = np.full((len(context_records), q_len, topk), -1, np.int32)
    lens = np.zeros((len(context_records), q_len), np.int32)
    for b, c in enumerate(context_records):
        n = min(topk, c)
        for s in range(q_len):
            idx[b, s, :n] = rng.choice(c, n, replace=False)
            lens[b, s] = n
    return idx, lens.reshape(-1)


def log_uniform_contexts(batch: int, lo_tokens: int, hi_tokens: int, seed: int):
    rng = np.random.default_rng(seed)
    tokens = np.exp(rng.uniform(math.log(lo_tokens), math.log(hi_tokens), batch))
    return [int(t) // 4 for t in tokens]  # C4: one record per 4 tokens


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a = a.astype(np.float64).ravel()
    b = b.astype(np.float64).ravel()
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na == 0 and nb == 0:
        return 1.0
    return float(a @ b / (na * nb))
