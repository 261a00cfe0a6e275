"""Seeded synthetic inputs shared by the fixture writer, the tests and bench.py.

Everything is drawn from the torch CPU generator, so the same seed gives the
same tensor on any machine running this image. Only the recipe and the seeds
are committed; the arrays are regenerated where they are needed.
"""
from __future__ import annotations

import numpy as np
import torch


def gaussian_weight(rows: int, cols: int, seed: int, sigma: float = 0.02,
                    outlier_frac: float = 0.001, outlier_gain: float = 20.0,
                    dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """N(0, sigma) weights with `outlier_frac` of positions scaled by `outlier_gain`."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(rows, cols, generator=g) * sigma
    n_hot = int(rows * cols * outlier_frac)
    if n_hot > 0:
        idx = torch.randperm(rows * cols, generator=g)[:n_hot]
        w.view(-1)[idx] *= outlier_gain
    return w.to(dtype)


def student_t_weight(rows: int, cols: int, seed: int, df: int = 5, sigma: float = 0.02,
                     dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Student-t(df) x sigma weights: z / sqrt(chi2_df / df).

    The square root is numpy's (IEEE, correctly rounded): torch's vectorized
    CPU sqrt is not, and its vector/scalar split depends on the thread count,
    so it gives different bits on hosts with different core counts."""
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(rows, cols, generator=g)
    c = torch.zeros(rows, cols)
    for _ in range(df):
        c += torch.randn(rows, cols, generator=g) ** 2
    root = torch.from_numpy(np.sqrt((c / df).numpy()))
    return (z / root * sigma).to(dtype)


def tie_heavy_weight(rows: int, cols: int, seed: int, levels: int = 64,
                     dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """Weights drawn from a small discrete set, so the top-k threshold is
    shared by many positions (exercises the top-k tie order)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-levels, levels + 1, (rows, cols), generator=g).to(torch.float32)
    return (q / levels * 0.05).to(dtype)


def activations(m: int, k: int, seed: int = 7, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """Activations x ~ N(0, 1) in bf16."""
    g = torch.Generator().manual_seed(seed)
    return torch.randn(m, k, generator=g).to(dtype)


# Llama-3-8B-shaped decoder-layer linears: (name, out_features, in_features).
LLAMA3_8B_LINEARS = (
    ("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
    ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336),
)

# Llama-3-70B-shaped layer linears.
LLAMA3_70B_LINEARS = (
    ("q", 8192, 8192), ("k", 1024, 8192), ("v", 1024, 8192), ("o", 8192, 8192),
    ("gate", 28672, 8192), ("up", 28672, 8192), ("down", 8192, 28672),
)


def layer_seed(index: int) -> int:
    """Seed for linear number `index` (q, k, v, o, gate, up, down = 0..6)."""
    return 1000 + index


def tiny_model(seed: int = 11):
    """A small decoder-shaped module tree for the module-level API tests:
    eligible linears (q/up/down in two blocks, mixed weight distributions so
    that the adaptive chain lands on different bit widths) next to ones the
    default skip rules exclude by name (norm, embed, lm_head) or size
    (numel < 16384). fp16 weights from the torch CPU generator."""
    import torch.nn as nn

    d, f = 256, 512

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = nn.Linear(d, d, bias=False)
            self.up_proj = nn.Linear(d, f, bias=True)
            self.down_proj = nn.Linear(f, d, bias=False)
            self.input_norm = nn.Linear(d, d, bias=False)

    class Tiny(nn.Module):
        def __init__(self):
            super().__init__()
            self.embed_tokens = nn.Linear(d, d, bias=False)
            self.layers = nn.ModuleList([Block(), Block()])
            self.lm_head = nn.Linear(d, 64, bias=False)
            self.tiny = nn.Linear(32, 32)

    m = Tiny()
    g = torch.Generator().manual_seed(seed)
    for i, (name, mod) in enumerate(sorted(m.named_modules(), key=lambda t: t[0])):
        if not isinstance(mod, nn.Linear):
            continue
        n, k = mod.weight.shape
        if "up_proj" in name:  # heavy tails: 4-bit error above typical thresholds
            w = student_t_weight(n, k, seed * 100 + i)
        elif "q_proj" in name and name.startswith("layers.1"):  # few distinct levels: 2-bit suffices
            w = tie_heavy_weight(n, k, seed * 100 + i, levels=2)
        else:
            w = gaussian_weight(n, k, seed * 100 + i)
        mod.weight.data = w.to(torch.float16)
        if mod.bias is not None:
            mod.bias.data = (torch.randn(n, generator=g) * 0.05).to(torch.float16)
    return m
