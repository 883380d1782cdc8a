"""Seeded synthetic inputs for the temporal-attention configurations.

Every tensor is drawn from ``torch.Generator``s seeded from ``seed`` in a fixed order, so the
same call gives the same inputs on every run. Small workloads are drawn on the CPU and
copied to ``device`` (the CPU checker then sees identical values); the large feature tables
of the multi-layer workloads are drawn directly on ``device``.

Distributions (the reference's training data are not available offline):
node / edge features ~ N(0, 1); dt = root time - neighbour time ~ Exp(mean 1e4);
upstream gradients ~ N(0, 1).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np
import torch

from .tgat import Block

DT_MEAN = 1e4


def _gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def ragged_degrees(num_dst: int, seed: int, s: float = 1.5, dmax: int = 20,
                   empty_frac: float = 0.05) -> np.ndarray:
    """Per-destination degrees clip(Zipf(s), 1, dmax) with ``empty_frac`` of the
    destinations set to 0 (numpy Generator, seeded)."""
    rng = np.random.default_rng(seed)
    deg = np.clip(rng.zipf(s, num_dst), 1, dmax).astype(np.int64)
    n_empty = int(round(empty_frac * num_dst))
    if n_empty:
        deg[rng.choice(num_dst, n_empty, replace=False)] = 0
    return deg


@dataclass
class LayerInputs:
    block: Block
    dout: torch.Tensor                      # upstream gradient [N, dim_out]
    dims: tuple                             # (Dn, De, Dt, H, D)


def single_layer(num_dst: int, fanout: int = 10, dn: int = 100, de: int = 172, dt_dim: int = 100,
                 heads: int = 2, dim_out: int = 100, seed: int = 0, device="cpu",
                 degrees: Optional[np.ndarray] = None, h_requires_grad: bool = False) -> LayerInputs:
    """One layer with dense, already gathered inputs (what ``prepare_input`` produces,
    utils.py:126-196): h [N+E, Dn], f [E, De], dt [E]. Fixed fanout unless ``degrees``."""
    if degrees is None:
        degrees = np.full(num_dst, fanout, dtype=np.int64)
    blk = Block.from_fanout(num_dst, torch.from_numpy(np.asarray(degrees, dtype=np.int64)))
    E = blk.num_edges()
    g = _gen(seed)
    dt = torch.empty(E).exponential_(1.0 / DT_MEAN, generator=g)
    h = torch.randn(num_dst + E, dn, generator=g)
    f = torch.randn(E, de, generator=g)
    dout = torch.randn(num_dst, dim_out, generator=g)
    blk.srcdata["h"] = h
    blk.edata["f"] = f
    blk.edata["dt"] = dt
    blk = blk.to(device)
    if h_requires_grad:
        blk.srcdata["h"].requires_grad_(True)
    return LayerInputs(blk, dout.to(device), (dn, de, dt_dim, heads, dim_out))


@dataclass
class StackInputs:
    blocks: List[Block]
    dout: torch.Tensor
    node_table: torch.Tensor
    edge_table: torch.Tensor
    dims: tuple
    edges_per_layer: List[int] = field(default_factory=list)


def two_layer(roots: int = 4000, fanout=(10, 10), n_nodes: int = 1_000_000,
              n_edge_rows: int = 10_000_000, dn: int = 100, de: int = 172, dt_dim: int = 100,
              heads: int = 2, dim_out: int = 100, seed: int = 0, device="cpu",
              hot_frac: float = 0.0, hot_share: float = 0.0,
              dtype=torch.float32, row_align: int = 1) -> StackInputs:
    """Two-layer TGAT MFG in the reference sampler's shape (modules.py:48-64, sampler_core
    re-sampling every source of the layer above): the top block has N1 = 3*roots
    destinations and N1*fanout[1] edges; the bottom block's destinations are all N1 + E1
    sources of the top block, each with fanout[0] edges. Node rows come from a node table
    (n_nodes x dn) and edge rows from an edge table (n_edge_rows x de), gathered by
    uniform random ids (``hot_share`` of them drawn from a ``hot_frac`` hot set). Table
    rows are allocated with a leading dimension rounded up to ``row_align`` elements."""
    N1 = 3 * roots
    E1 = N1 * fanout[1]
    N0 = N1 + E1
    E0 = N0 * fanout[0]
    gd = _gen(seed, device)

    def ids(n, high):
        if hot_share > 0:
            hot = max(1, int(hot_frac * high))
            r = torch.randint(0, high, (n,), generator=gd, device=device)
            hsel = torch.rand(n, generator=gd, device=device) < hot_share
            hr = torch.randint(0, hot, (n,), generator=gd, device=device)
            return torch.where(hsel, hr, r)
        return torch.randint(0, high, (n,), generator=gd, device=device)

    def table(n, d):
        ld = -(-d // row_align) * row_align
        return torch.randn(n, ld, generator=gd, device=device, dtype=dtype)[:, :d]

    node_table = table(n_nodes, dn)
    edge_table = table(n_edge_rows, de)
    b0 = Block.from_fanout(N0, torch.full((N0,), fanout[0], dtype=torch.int64, device=device))
    b0.node_table = node_table
    b0.edge_table = edge_table
    b0.srcdata["ID"] = ids(N0 + E0, n_nodes)
    b0.edata["ID"] = ids(E0, n_edge_rows)
    b0.edata["dt"] = torch.empty(E0, device=device).exponential_(1.0 / DT_MEAN, generator=gd)
    b1 = Block.from_fanout(N1, torch.full((N1,), fanout[1], dtype=torch.int64, device=device))
    b1.edge_table = edge_table
    b1.edata["ID"] = ids(E1, n_edge_rows)
    b1.edata["dt"] = torch.empty(E1, device=device).exponential_(1.0 / DT_MEAN, generator=gd)
    dout = torch.randn(N1, dim_out, generator=gd, device=device)
    return StackInputs([b0, b1], dout, node_table, edge_table, (dn, de, dt_dim, heads, dim_out),
                       [E0, E1])


def ragged_layer(num_dst: int = 200_000, n_nodes: int = 1_000_000, n_edge_rows: int = 10_000_000,
                 dn: int = 100, de: int = 172, dt_dim: int = 100, heads: int = 2,
                 dim_out: int = 100, seed: int = 0, device="cpu") -> LayerInputs:
    """Recent-neighbour sampling truncated by history length: ragged Zipf(1.5) degrees in
    [1, 20] with 5 % empty destinations; node rows from a memory table, edge rows from an
    edge table, both gathered by uniform random ids."""
    deg = ragged_degrees(num_dst, seed)
    blk = Block.from_fanout(num_dst, torch.from_numpy(deg).to(device))
    E = blk.num_edges()
    gd = _gen(seed, device)
    blk.node_table = torch.randn(n_nodes, dn, generator=gd, device=device)
    blk.edge_table = torch.randn(n_edge_rows, de, generator=gd, device=device)
    blk.srcdata["ID"] = torch.randint(0, n_nodes, (num_dst + E,), generator=gd, device=device)
    blk.edata["ID"] = torch.randint(0, n_edge_rows, (E,), generator=gd, device=device)
    blk.edata["dt"] = torch.empty(E, device=device).exponential_(1.0 / DT_MEAN, generator=gd)
    dout = torch.randn(num_dst, dim_out, generator=gd, device=device)
    return LayerInputs(blk, dout, (dn, de, dt_dim, heads, dim_out))
