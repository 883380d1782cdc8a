"""TGAT temporal attention on the fused gfx950 kernels.

``TransfomerAttentionLayer`` has the constructor, parameters (names, shapes, creation
order, initialisation) and ``forward(b, _layers, _hist)`` of the reference layer
(layers.py:53-240, TGAT/TGN branch) and computes the same function. Its data path differs:

  reference                                   this layer
  K = w_k(cat[h_src, f, cos(w dt+b)])  [E,D]  qt[h,v] = Q[v,h] W_k[h] (+ b_k column)   [H,N,Kp]
  V = w_v(cat[...])                    [E,D]  xbar[h,v] = sum_e a'[e,h] x_e (one kernel) [H,N,Kp]
  score = sum(Q[dst]*K), softmax, V*att,      agg[v,h] = W_v[h] xbar[h,v]               [N,D]
  update_all(copy_u, sum), w_out              rst = w_out([agg | h_dst])

so the K/V projections run over the N destinations instead of the E edges, one head at a
time (Q[v,h] has D/H entries, so the per-head products cost D*Kp per destination, where
one folded product over all heads would cost H*D*Kp), and the neighbour gather, time
encoding, scoring, segment softmax and weighted reduction happen in one pass over the
gathered rows x_e (never written to memory). The per-head products run on the matrix
cores (fastAgg.head_proj / head_reduce / head_wgrad), head-major so that each head's
block [N, Kp] is contiguous.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from . import fastAgg


# ---------------------------------------------------------------------------------------
# Message-flow-graph block
# ---------------------------------------------------------------------------------------
class Block:
    """Destination-sorted bipartite block with the subset of the DGL block API that the
    TGAT layer uses (``num_dst_nodes``, ``num_src_nodes``, ``num_edges``, ``edges``,
    ``srcdata``, ``dstdata``, ``edata``).

    Layout contract of the FAST sampler (sampler_core.cpp:159-181, 185-456; utils.py:67-87):
    source nodes ``0..N-1`` are the destinations themselves and edge ``e`` comes from source
    node ``N + e``; edges are grouped by ascending destination.

    Node features come either from ``srcdata['h']`` (dense, one row per source node) or
    from ``node_table`` gathered by ``srcdata['ID']``; edge features from ``edata['f']`` or
    ``edge_table`` gathered by ``edata['ID']``. ``indptr`` optionally holds the sampler's
    compressed int32 CSR (``cntE``).
    """

    def __init__(self, src: torch.Tensor, dst: torch.Tensor, num_src: int, num_dst: int,
                 indptr: Optional[torch.Tensor] = None):
        self._src = src
        self._dst = dst
        self._num_src = int(num_src)
        self._num_dst = int(num_dst)
        self.indptr = indptr
        self.srcdata: dict = {}
        self.dstdata: dict = {}
        self.edata: dict = {}
        self.node_table: Optional[torch.Tensor] = None
        self.edge_table: Optional[torch.Tensor] = None
        self._rowptr: Optional[torch.Tensor] = None

    @classmethod
    def from_fanout(cls, num_dst: int, degrees: torch.Tensor) -> "Block":
        """Block in the sampler layout for per-destination degrees (int64 [num_dst])."""
        dev = degrees.device
        dst = torch.repeat_interleave(torch.arange(num_dst, device=dev), degrees)
        E = int(dst.numel())
        src = torch.arange(num_dst, num_dst + E, device=dev)
        counts = degrees[degrees > 0].to(torch.int64)
        indptr = torch.zeros(counts.numel() + 1, dtype=torch.int32, device=dev)
        if counts.numel():
            indptr[1:] = torch.cumsum(counts, 0).to(torch.int32)
        return cls(src, dst, num_dst + E, num_dst, indptr)

    def num_dst_nodes(self) -> int:
        return self._num_dst

    def num_src_nodes(self) -> int:
        return self._num_src

    def num_edges(self) -> int:
        return int(self._dst.numel())

    def edges(self):
        return self._src, self._dst

    @property
    def device(self) -> torch.device:
        return self._dst.device

    def rowptr(self) -> torch.Tensor:
        """int32 [N+1] offsets of every destination's edges (zero-degree ones included)."""
        if self._rowptr is None:
            self._rowptr = fastAgg.rowptr_from_dst(self._dst, self._num_dst)
        return self._rowptr

    def to(self, device) -> "Block":
        def mv(t):
            return t.to(device) if isinstance(t, torch.Tensor) else t
        b = Block(mv(self._src), mv(self._dst), self._num_src, self._num_dst, mv(self.indptr))
        b.srcdata = {k: mv(v) for k, v in self.srcdata.items()}
        b.dstdata = {k: mv(v) for k, v in self.dstdata.items()}
        b.edata = {k: mv(v) for k, v in self.edata.items()}
        b.node_table = mv(self.node_table)
        b.edge_table = mv(self.edge_table)
        return b

    # -- feature access -----------------------------------------------------------------
    def dst_node_feats(self, pad4: bool = False) -> Optional[torch.Tensor]:
        """The destination rows' node features [N, Dn]; with ``pad4`` and a gathered table,
        [N, Dn rounded up to 4] with zero columns past Dn (rows in whole 16-byte chunks)."""
        N = self._num_dst
        if "h" in self.srcdata:
            return self.srcdata["h"][:N]
        if self.node_table is not None:
            ids = self.srcdata["ID"][:N]
            width = -(-self.node_table.shape[1] // 4) * 4 if pad4 else 0
            return fastAgg.gather_rows(self.node_table, ids, N, width)
        return None

    def src_node_source(self):
        """(table, per-edge row index or None) of the node rows feeding the edges."""
        N = self._num_dst
        if "h" in self.srcdata:
            return self.srcdata["h"][N:], None
        if self.node_table is not None:
            return self.node_table, self.srcdata["ID"][N:]
        return None, None

    def edge_source(self):
        if "f" in self.edata:
            return self.edata["f"], None
        if self.edge_table is not None:
            return self.edge_table, self.edata["ID"]
        return None, None


# ---------------------------------------------------------------------------------------
# Time encoding
# ---------------------------------------------------------------------------------------
def time_encoding_weight(dim: int) -> torch.Tensor:
    """w_j = 1 / 10**linspace(0, 9, dim) in float32, shape [dim, 1] (layers.py:14)."""
    return torch.from_numpy(1 / 10 ** np.linspace(0, 9, dim, dtype=np.float32)).reshape(dim, -1)


class TimeEncode(torch.nn.Module):
    """cos(w * t + b) with w, b trainable (layers.py:8-29). The argument is evaluated as a
    rounded product followed by a rounded sum, the same as the fused kernels."""

    def __init__(self, dim: int):
        super().__init__()
        self.dim = dim
        self.w = torch.nn.Linear(1, dim)
        self.w.weight = torch.nn.Parameter(time_encoding_weight(dim))
        self.w.bias = torch.nn.Parameter(torch.zeros(dim))

    def forward(self, t: torch.Tensor) -> torch.Tensor:
        return torch.cos(t.reshape(-1, 1) * self.w.weight.view(1, -1) + self.w.bias)


# ---------------------------------------------------------------------------------------
# K-space helpers
# ---------------------------------------------------------------------------------------
def kspace_width(dn: int, de: int, dt: int) -> int:
    return int(fastAgg.tgat_kspace(dn, de, dt))


_KSPACE_COLS: dict = {}


def kspace_columns(dn: int, de: int, dt: int, device) -> torch.Tensor:
    """Column of the K-space layout that holds each of the dn+de+dt input columns (node,
    edge and time parts each padded to a multiple of 4); cached per shape and device."""
    key = (dn, de, dt, str(device))
    cols = _KSPACE_COLS.get(key)
    if cols is None:
        idx, off = [], 0
        for d in (dn, de, dt):
            idx.extend(range(off, off + d))
            off += d + (-d) % 4
        cols = torch.tensor(idx, dtype=torch.long, device=device)
        _KSPACE_COLS[key] = cols
    return cols


class _ToKspace(torch.autograd.Function):
    @staticmethod
    def forward(ctx, W, b, dn, de, dt):
        kp = kspace_width(dn, de, dt)
        cols = kspace_columns(dn, de, dt, W.device)
        kb = 4 * ((dn + 3) // 4 + (de + 3) // 4 + (dt + 3) // 4)
        out = W.new_zeros(W.shape[0], kp)
        out.index_copy_(1, cols, W)
        out[:, kb] = b
        ctx.cols, ctx.kb = cols, kb
        return out

    @staticmethod
    def backward(ctx, dout):
        dW = dout.index_select(1, ctx.cols) if ctx.needs_input_grad[0] else None
        db = dout[:, ctx.kb].contiguous() if ctx.needs_input_grad[1] else None
        return dW, db, None, None, None


def to_kspace(W: torch.Tensor, b: torch.Tensor, dn: int, de: int, dt: int) -> torch.Tensor:
    """[D, dn+de+dt] weight and [D] bias -> [D, Kp] with each part padded to a multiple of
    4 columns, the bias at column Kb and zeros after it (the layout the kernels use). One
    scatter forward and one gather backward."""
    return _ToKspace.apply(W, b, dn, de, dt)


def fused_kernel_bytes(n_dst: int, n_edges: int, dn: int, de: int, dt: int, heads: int,
                       node_idx: bool, edge_idx: bool, d_node: bool = False,
                       node_bytes: int = 4, edge_bytes: int = 4, tdot: bool = False) -> dict:
    """Algorithmic HBM bytes of one launch of the fused forward / backward kernel (float32):
    every byte the kernel must read or write once, gathered rows counted once per use.

    per edge : node id (8, when gathered) + edge id (8, when gathered) + dt (4)
               + node row (node_bytes*dn) + edge row (edge_bytes*de)
               + score (4*heads, written / read)
               [+ d_node row (4*dn) written in backward when requested]
    per dst  : forward  qt read + xbar written (2 * 4*heads*Kp) + stats written (8*heads)
               backward dxbar, xbar read + dqt written (3 * 4*heads*Kp) + stats read (8*heads)
               + the qt chunks the backward uses (4*heads*4*(ct + cn with d_node): the time
               part, and the node part when the node-row gradient is written);
               with ``tdot`` the per-head dot products (4*heads) are read instead of xbar
    plus the row offsets 4*(n_dst+1) and the time parameters 8*dt."""
    kp = kspace_width(dn, de, dt)
    edge_in = (8 if node_idx else 0) + (8 if edge_idx else 0) + 4 + node_bytes * dn + edge_bytes * de
    common = 4 * (n_dst + 1) + 8 * dt
    fwd = common + n_edges * (edge_in + 4 * heads) + n_dst * (2 * 4 * heads * kp + 8 * heads)
    q_read = 16 * heads * ((dt + 3) // 4 + ((dn + 3) // 4 if d_node else 0))
    dst_rows = q_read + ((2 * 4 * heads * kp + 4 * heads) if tdot else 3 * 4 * heads * kp)
    bwd = (common + n_edges * (edge_in + 4 * heads + (4 * dn if d_node else 0))
           + n_dst * (dst_rows + 8 * heads))
    return {"fwd": fwd, "bwd": bwd}


class KernelTimer:
    """Records a HIP event pair around every fused-kernel call on torch's current stream
    (the stream the kernels are enqueued on) with the launch's algorithmic bytes."""

    def __init__(self):
        self.records = []   # (name, start_event, end_event, bytes)
        self.enabled = True

    def begin(self):
        if not self.enabled:
            return None
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        return ev

    def end(self, name, start, nbytes):
        if start is None:
            return
        ev = torch.cuda.Event(enable_timing=True)
        ev.record()
        self.records.append((name, start, ev, nbytes))

    def reset(self):
        self.records = []

    def summary(self) -> dict:
        """Per kernel: launches, total ms, total algorithmic bytes, GB/s (call after a
        device synchronisation)."""
        out = {}
        for name, s, e, nb in self.records:
            d = out.setdefault(name, {"launches": 0, "ms": 0.0, "bytes": 0})
            d["launches"] += 1
            d["ms"] += s.elapsed_time(e)
            d["bytes"] += nb
        for d in out.values():
            d["GB/s"] = d["bytes"] / (d["ms"] * 1e-3) / 1e9 if d["ms"] > 0 else 0.0
            d["avg_us"] = 1e3 * d["ms"] / max(1, d["launches"])
        return out


timer: Optional[KernelTimer] = None  # set by a benchmark to time the fused kernels


def _timed(name: str, nbytes: int, fn, *args):
    """fn(*args), bracketed by timer events with its algorithmic bytes when a timer is set."""
    t0 = timer.begin() if timer is not None else None
    out = fn(*args)
    if t0 is not None:
        timer.end(name, t0, nbytes)
    return out


def _head_bytes(n: int, g: int, j: int, c: int, x_groups: bool = True) -> int:
    """Algorithmic bytes of a per-head product over an [n, g*j] side and a [g, n, c] block:
    both read or written once (the [g, n, c] side once per group unless it is one array
    shared by every group, x_groups False), plus the [g, j, c] weights."""
    return 4 * (n * g * j + (g if x_groups else 1) * n * c + g * j * c)
# When set to a list, each layer's forward appends its post-activation values, whose signs
# are the branches its backward takes: ("score", [E, H] post-LeakyReLU scores) from the fused
# kernel, then ("relu", [N, D] post-dropout, post-ReLU values) from the epilogue. A parity
# test reads them.
branch_sink: Optional[list] = None


class _Graph:
    """Non-differentiable per-block operands of the fused kernels."""

    __slots__ = ("rowptr", "node_idx", "edge_tab", "edge_idx", "dt", "node_front")

    def __init__(self, rowptr, node_idx, edge_tab, edge_idx, dt, node_front: int = 0):
        self.rowptr = rowptr
        self.node_idx = node_idx
        self.edge_tab = edge_tab
        self.edge_idx = edge_idx
        self.dt = dt
        # rows of the source tensor in front of the edge rows (the destination rows, when the
        # edge rows are h[N:] of a dense h): the backward leaves them free in front of the
        # edge-row gradient so that the two gradients form one tensor without a copy
        self.node_front = node_front


class TgatAttention(torch.autograd.Function):
    """xbar = fused gather/time-encode/score/softmax/reduce (see module docstring).

    Differentiable inputs: ``qt`` [H,N,Kp], ``time_w`` [Dt], ``time_b`` [Dt] and
    ``node_src`` (the node rows feeding the edges: one row per edge when ``node_idx`` is
    None, else a table gathered by ``node_idx``)."""

    @staticmethod
    def forward(ctx, qt, time_w, time_b, node_src, g: _Graph, slope: float, drop,
                drop_seed: int = 0, drop_p: float = 0.0, link: Optional["_TdotLink"] = None):
        t0 = timer.begin() if timer is not None else None
        xbar, scores, stats = fastAgg.tgat_attn_fwd(g.rowptr, node_src, g.node_idx, g.edge_tab,
                                                    g.edge_idx, g.dt, time_w, time_b, qt,
                                                    float(slope), drop, int(drop_seed),
                                                    float(drop_p))
        if t0 is not None:
            nb = fused_kernel_bytes(qt.shape[1], g.dt.numel(), node_src.shape[1],
                                    g.edge_tab.shape[1], time_w.numel(), qt.shape[0],
                                    g.node_idx is not None, g.edge_idx is not None,
                                    node_bytes=node_src.element_size(),
                                    edge_bytes=g.edge_tab.element_size())["fwd"]
            timer.end("tgat_fwd", t0, nb)
        if branch_sink is not None:
            branch_sink.append(("score", scores))
        ctx.g = g
        ctx.link = link
        ctx.slope = float(slope)
        ctx.has_drop = drop is not None
        ctx.drop_seed = int(drop_seed)
        ctx.drop_p = float(drop_p)
        saved = [qt, time_w, time_b, node_src, xbar, scores, stats]
        if drop is not None:
            saved.append(drop)
        ctx.save_for_backward(*saved)
        return xbar

    @staticmethod
    def backward(ctx, dxbar):
        saved = ctx.saved_tensors
        qt, time_w, time_b, node_src, xbar, scores, stats = saved[:7]
        drop = saved[7] if ctx.has_drop else None
        g = ctx.g
        need_node = ctx.needs_input_grad[3] and node_src.shape[1] > 0
        if dxbar.stride(2) != 1:   # the kernel takes any row / head strides
            dxbar = dxbar.contiguous()
        # dxbar . xbar per destination and head, when the consumer of xbar supplied it
        tdot = ctx.link.take() if ctx.link is not None else None
        t0 = timer.begin() if timer is not None else None
        dqt, d_node, d_tw, d_tb = fastAgg.tgat_attn_bwd(g.rowptr, node_src, g.node_idx,
                                                        g.edge_tab, g.edge_idx, g.dt, time_w,
                                                        time_b, qt, ctx.slope, drop,
                                                        ctx.drop_seed, ctx.drop_p,
                                                        None if tdot is not None else xbar,
                                                        scores, stats, dxbar, need_node, tdot,
                                                        g.node_front if g.node_idx is None else 0)
        if t0 is not None:
            nb = fused_kernel_bytes(qt.shape[1], g.dt.numel(), node_src.shape[1],
                                    g.edge_tab.shape[1], time_w.numel(), qt.shape[0],
                                    g.node_idx is not None, g.edge_idx is not None,
                                    need_node, node_bytes=node_src.element_size(),
                                    edge_bytes=g.edge_tab.element_size(),
                                    tdot=tdot is not None)["bwd"]
            timer.end("tgat_bwd", t0, nb)
        d_src = None
        if need_node:
            if g.node_idx is None:
                d_src = d_node
            else:
                d_src = torch.zeros_like(node_src).index_add_(0, g.node_idx, d_node)
        return dqt, d_tw, d_tb, d_src, None, None, None, None, None, None


class _TdotLink:
    """Carries T[v, h] = dxbar[h, v] . xbar[h, v] from the backward of the reduction that
    consumes xbar (HeadReduce: with agg = W_v xbar, T = dagg . agg over D/H entries instead
    of Kp) to the backward of TgatAttention, which runs right after it."""

    def __init__(self):
        self.tdot = None

    def take(self):
        t, self.tdot = self.tdot, None
        return t


# Widest head (J) the per-head product kernels take (fastAgg.head_proj / head_reduce hold a
# head's J x C weight fragments in registers); wider heads use batched float32 GEMMs.
HEAD_KERNEL_MAX_J = 64


def _proj(x, w, bias):
    """[N, G*J] x [G, J, C] (+ [G, C]) -> [G, N, C]."""
    G, J, C = w.shape
    if J <= HEAD_KERNEL_MAX_J:
        return _timed("head_proj", _head_bytes(x.shape[0], G, J, C), fastAgg.head_proj, x, w, bias)
    y = torch.matmul(x.view(-1, G, J).transpose(0, 1), w)
    return y if bias is None else y + bias[:, None, :]


def _rows16(t) -> bool:
    """Rows of whole 16-byte chunks: 16-byte aligned, unit inner stride, other strides and
    the width multiples of 4 (the split-bf16 kernels' condition)."""
    return (t.data_ptr() % 16 == 0 and t.stride(-1) == 1 and t.shape[-1] % 4 == 0
            and all(st % 4 == 0 for st in t.stride()[:-1]))


def _reduce_path(y, J: int) -> int:
    """The head_reduce kernel path for y [G, N, C] and heads of width J (0: none)."""
    if J > HEAD_KERNEL_MAX_J or y.stride(-1) != 1:
        return 0
    return int(fastAgg.head_reduce_supported(J, y.shape[2], y.stride(1), _rows16(y)))


def _reduce(y, w, name: str = "head_reduce"):
    """[G, N, C] x [G, J, C]^T -> [N, G*J]; batched torch GEMMs where the head kernel does
    not take the shape (heads wider than 64, or W[g] too large for LDS). Timed as ``name``."""
    G, J, C = w.shape
    if _reduce_path(y, J):
        return _timed(name, _head_bytes(y.shape[1], G, J, C, y.stride(0) != 0),
                      fastAgg.head_reduce, y, w)
    z = torch.matmul(y, w.transpose(1, 2).contiguous())
    return z.transpose(0, 1).reshape(y.shape[1], G * J)


def _wgrad(x, y, groups: int, ones: bool):
    """fastAgg.head_wgrad (dw[g] = x[:, g-block]^T y[g], plus the column sums of y[g] with
    ``ones``), timed as head_wgrad: x [N, G*J] and y [G, N, C] read once, dw written."""
    G, n, C = y.shape
    J = x.shape[1] // groups
    nb = 4 * (n * groups * J + (G if y.stride(0) != 0 else 1) * n * C + groups * (J + int(ones)) * C)
    return _timed("head_wgrad", nb, fastAgg.head_wgrad, x, y, groups, ones)


def _rows_mm(x, a, name: str = "head_reduce"):
    """x @ a^T for x [N, K] with many rows and a small a [M, K]: the per-head reduce kernel
    with every group reading the same rows of x (fastAgg.head_reduce with a zero group
    stride; M split into G groups of at most HEAD_KERNEL_MAX_J rows of a), used where its
    split-bf16 form applies (rows of x in whole 16-byte chunks); torch's GEMM otherwise.
    Timed as ``name``."""
    m, k = a.shape
    if x.dim() != 2 or x.stride(1) != 1 or k % 4 or x.stride(0) % 4 or x.data_ptr() % 16:
        return x @ a.t()
    # the fewest groups (widest heads, at most 64 rows of a each) that the split-bf16 kernel
    # takes, else that the float32 kernel takes, else torch's GEMM
    xs = x.unsqueeze(0).expand(1, x.shape[0], k)
    cands = [d for d in range(1, m + 1) if m % d == 0 and m // d <= HEAD_KERNEL_MAX_J]
    g = next((d for d in cands if _reduce_path(xs, m // d) == 2), None)
    if g is None:
        g = next((d for d in cands if _reduce_path(xs, m // d) == 1), None)
    if g is None:
        return x @ a.t()
    a = a.contiguous()
    return _reduce(x.unsqueeze(0).expand(g, x.shape[0], k), a.view(g, m // g, k), name)


class _SplitRows(torch.autograd.Function):
    """(h[:n], h[n:]): the destination rows and the rows feeding the edges of a dense
    source-feature tensor. Its backward concatenates the two gradients into one tensor (two
    plain slices would each zero-fill a full-size gradient and then add them)."""

    @staticmethod
    def forward(ctx, h, n: int):
        ctx.n = int(n)
        ctx.shape = h.shape
        return h[:n], h[n:]

    @staticmethod
    def backward(ctx, g_dst, g_src):
        n, (rows, dim) = ctx.n, ctx.shape
        base = g_src._base if g_src is not None else None
        if (g_dst is not None and base is not None and base.shape == (rows, dim)
                and base.is_contiguous() and g_src.data_ptr() == base[n:].data_ptr()):
            # the fused backward wrote g_src into rows n.. of a full-size tensor (its
            # d_node_front): fill the rows in front instead of concatenating
            base[:n].copy_(g_dst)
            return base, None
        if g_dst is None:
            g_dst = torch.zeros(n, dim, device=g_src.device, dtype=g_src.dtype)
        if g_src is None:
            g_src = torch.zeros(rows - n, dim, device=g_dst.device, dtype=g_dst.dtype)
        return torch.cat([g_dst, g_src]), None


class HeadProj(torch.autograd.Function):
    """y[g] = x[:, g*J:(g+1)*J] @ w[g] (+ bias[g]) for x [N, G*J], w [G, J, C] -> [G, N, C]."""

    @staticmethod
    def forward(ctx, x, w, bias):
        ctx.save_for_backward(x, w)
        ctx.has_bias = bias is not None
        return _proj(x, w, bias)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = _reduce(dy, w)
        if ctx.needs_input_grad[1] or (ctx.has_bias and ctx.needs_input_grad[2]):
            gw = _wgrad(x, dy, w.shape[0], ctx.has_bias)
            dw = gw[:, :w.shape[1]]
            db = gw[:, w.shape[1]] if ctx.has_bias else None
        return dx, dw, db


class HeadReduce(torch.autograd.Function):
    """z[:, g*J:(g+1)*J] = y[g] @ w[g]^T for y [G, N, C], w [G, J, C] -> [N, G*J]. With a
    ``link``, its backward also leaves T[n, g] = dy[g, n] . y[g, n] = dz[n, g-block] .
    z[n, g-block] there (for TgatAttention's backward)."""

    @staticmethod
    def forward(ctx, y, w, link: Optional[_TdotLink] = None):
        z = _reduce(y, w)
        ctx.link = link
        ctx.save_for_backward(y, w, z)
        return z

    @staticmethod
    def backward(ctx, dz):
        y, w, z = ctx.saved_tensors
        dz = dz.contiguous()
        # the weight gradient first: dy, written last, is what the next kernel (the fused
        # backward) reads, so its most recent part is still in the last-level cache
        dw = _wgrad(dz, y, w.shape[0], False) if ctx.needs_input_grad[1] else None
        dy = _proj(dz, w, None) if ctx.needs_input_grad[0] else None
        if ctx.link is not None and dy is not None:
            ctx.link.tdot = fastAgg.row_group_dots(dz, z, w.shape[0])
        return dy, dw, None


class TgatEpilogue(torch.autograd.Function):
    """LayerNorm(ReLU(dropout(r1 + r2 + bias))) in one kernel each way (layers.py:235-236);
    the dropout is the counter hash of (seed, row*d + col), as fastAgg.dropout_mask."""

    @staticmethod
    def forward(ctx, r1, r2, bias, gamma, beta, eps: float, seed: int, p: float):
        out, y, stats = fastAgg.tgat_epilogue_fwd(r1, r2, bias, gamma, beta, float(eps),
                                                  int(seed), float(p))
        if branch_sink is not None:
            branch_sink.append(("relu", y))
        ctx.save_for_backward(y, stats, gamma)
        ctx.p = float(p)
        ctx.has_r2 = r2 is not None
        ctx.has_bias = bias is not None
        return out

    @staticmethod
    def backward(ctx, dout):
        y, stats, gamma = ctx.saved_tensors
        du, dgamma, dbeta, dbias = fastAgg.tgat_epilogue_bwd(dout.contiguous(), y, stats, gamma,
                                                             ctx.p, ctx.has_bias)
        return (du, (du if ctx.has_r2 else None), (dbias if ctx.has_bias else None), dgamma,
                dbeta, None, None, None)


class RowsMM(torch.autograd.Function):
    """y = x W^T for x [N, K] with many rows and a small W [M, K] (no bias), and dx = dy W,
    on the per-head reduce kernel (`_rows_mm`). The weight gradient x^T dy is the split-row
    reduction of fastAgg.head_wgrad (deterministic)."""

    @staticmethod
    def forward(ctx, x, W):
        ctx.save_for_backward(x, W)
        return _rows_mm(x, W)

    @staticmethod
    def backward(ctx, dy):
        x, W = ctx.saved_tensors
        dy = dy.contiguous()
        dx = _rows_mm(dy, W.t()) if ctx.needs_input_grad[0] else None
        dW = None
        if ctx.needs_input_grad[1]:   # dy^T x, written [M, K] (no transposed view)
            dW = _wgrad(dy, x.unsqueeze(0), 1, False)[0]
        return dx, dW


class DstProj(torch.autograd.Function):
    """The two products of the destination features in one GEMM:
    [q | r] = h [Wq | Wr]^T for h [N, K], Wq [Mq, K], Wr [Mr, K] (the query projection and
    the h_dst half of w_out), returned as two column blocks of one [N, Mq+Mr] array."""

    @staticmethod
    def forward(ctx, h, Wq, Wr):
        ctx.save_for_backward(h, Wq, Wr)
        t = _rows_mm(h, torch.cat([Wq, Wr], 0))
        mq = Wq.shape[0]
        return t[:, :mq], t[:, mq:]

    @staticmethod
    def backward(ctx, dq, dr):
        h, Wq, Wr = ctx.saved_tensors
        dh = dWq = dWr = None
        if dq is not None:
            dq = dq.contiguous()
        if dr is not None:
            dr = dr.contiguous()
        if ctx.needs_input_grad[0]:
            if dq is not None:
                dh = dq @ Wq
                if dr is not None:
                    dh.addmm_(dr, Wr)
            elif dr is not None:
                dh = dr @ Wr
        hc = h.contiguous() if (ctx.needs_input_grad[1] or ctx.needs_input_grad[2]) else h
        if ctx.needs_input_grad[1] and dq is not None:
            dWq = _wgrad(dq, hc.unsqueeze(0), 1, False)[0]
        if ctx.needs_input_grad[2] and dr is not None:
            dWr = _wgrad(dr, hc.unsqueeze(0), 1, False)[0]
        return dh, dWq, dWr


class LayerParams(torch.autograd.Function):
    """The layer's weights in the forms the step uses, one kernel each way
    (fastAgg.layer_params_fwd / _bwd): W_q[:, :Dn]; W_k and W_v with their biases in the
    K-space layout; qbk[h] = qb[h-block] W_k,aug[h-block] with the query bias
    qb = b_q + W_q[:, Dn:] cos(b_t) (layers.py:109-110); W_o[:, :D] and W_o[:, D:]."""

    @staticmethod
    def forward(ctx, wq, bq, wk, bk, wv, bv, bt, wo, dims):
        heads, dn, de, dt = dims
        ctx.dims = dims
        ctx.save_for_backward(wq, bq, wk, bk, bt if bt is not None else wq.new_empty(0))
        return tuple(fastAgg.layer_params_fwd(wq, bq, wk, bk, wv, bv, bt, wo, heads, dn, de, dt))

    @staticmethod
    def backward(ctx, g_wq, g_wk, g_wv, g_qbk, g_wo1, g_wo2):
        heads, dn, de, dt = ctx.dims
        wq, bq, wk, bk, bt = ctx.saved_tensors
        c = lambda t: t.contiguous() if t is not None else None
        d_wq, d_bq, d_wk, d_bk, d_wv, d_bv, d_bt, d_wo = fastAgg.layer_params_bwd(
            wq, bq, wk, bk, bt if dt > 0 else None, c(g_wq), c(g_wk), c(g_wv), c(g_qbk),
            c(g_wo1), c(g_wo2), heads, dn, de, dt)
        return d_wq, d_bq, d_wk, d_bk, d_wv, d_bv, (d_bt if dt > 0 else None), d_wo, None


# ---------------------------------------------------------------------------------------
# Layer
# ---------------------------------------------------------------------------------------
class TransfomerAttentionLayer(torch.nn.Module):
    """Temporal graph attention layer (layers.py:53-240), TGAT/TGN branch, on the fused
    kernels. The constructor creates the same modules in the same order as the reference,
    so a given seed yields the same initial weights and the state dicts are interchangeable.
    """

    def __init__(self, dim_node_feat, dim_edge_feat, dim_time, num_head, dropout, att_dropout,
                 dim_out, combined=False):
        super().__init__()
        if combined:
            raise NotImplementedError("the 'combined' projection variant is not built")
        if dim_out % num_head:
            raise ValueError("dim_out must be divisible by num_head")
        self.num_head = num_head
        self.dim_node_feat = dim_node_feat
        self.dim_edge_feat = dim_edge_feat
        self.dim_time = dim_time
        self.dim_out = dim_out
        self.dropout = torch.nn.Dropout(dropout)
        self.att_dropout = torch.nn.Dropout(att_dropout)
        self.negative_slope = 0.2
        self.att_act = torch.nn.LeakyReLU(self.negative_slope)
        self.combined = combined
        if dim_time > 0:
            self.time_enc = TimeEncode(dim_time)
        if dim_node_feat + dim_time > 0:
            self.w_q = torch.nn.Linear(dim_node_feat + dim_time, dim_out)
        self.w_k = torch.nn.Linear(dim_node_feat + dim_edge_feat + dim_time, dim_out)
        self.w_v = torch.nn.Linear(dim_node_feat + dim_edge_feat + dim_time, dim_out)
        self.w_out = torch.nn.Linear(dim_node_feat + dim_out, dim_out)
        self.layer_norm = torch.nn.LayerNorm(dim_out)

    def _query_bias(self) -> Optional[torch.Tensor]:
        """Bias of the query projection with the time encoding of dt = 0 for every
        destination folded in (layers.py:109-110): b_q + W_q[:, Dn:] cos(b)."""
        Dn, Dt = self.dim_node_feat, self.dim_time
        bias = self.w_q.bias
        if Dt > 0:
            bias = bias + torch.mv(self.w_q.weight[:, Dn:], torch.cos(self.time_enc.w.bias))
        return bias

    def forward(self, b: Block, _layers: int = 0, _hist: int = 0) -> torch.Tensor:
        # Dropout seeds of the kernels' counter-based masks, drawn from torch's CPU
        # generator, so torch.manual_seed makes a training run reproducible.
        kw = {}
        if self.training and self.att_dropout.p > 0:
            kw.update(drop_seed=int(torch.randint(0, 2**62, (1,)).item()), drop_p=self.att_dropout.p)
        if self.training and self.dropout.p > 0:
            kw.update(out_drop_seed=int(torch.randint(0, 2**62, (1,)).item()),
                      out_drop_p=self.dropout.p)
        return self.attend(b, **kw)

    def attend(self, b: Block, drop: Optional[torch.Tensor] = None, drop_seed: int = 0,
               drop_p: float = 0.0, out_drop_seed: int = 0, out_drop_p: float = 0.0) -> torch.Tensor:
        """The layer with explicit dropouts. Attention dropout: ``drop`` [E, heads]
        multipliers (0 or 1/(1-p) per entry), or, when ``drop`` is None and ``drop_p`` > 0,
        the kernels' hashed dropout of seed ``drop_seed``. Output dropout (before the ReLU):
        the hashed dropout of seed ``out_drop_seed`` over the [N, D] entries when
        ``out_drop_p`` > 0. fastAgg.dropout_mask gives the multipliers of either."""
        Dn, De, Dt = self.dim_node_feat, self.dim_edge_feat, self.dim_time
        H, D = self.num_head, self.dim_out
        dh = D // H
        N, E = b.num_dst_nodes(), b.num_edges()
        dev = b.device
        if E == 0:  # layers.py:101-102
            return torch.zeros((N, D), device=dev)
        node_src = node_idx = None
        if Dn > 0 and "h" in b.srcdata:
            hdst, node_src = _SplitRows.apply(b.srcdata["h"], N)
            if Dn % 4:   # rows in whole 16-byte chunks for the row products, as gathered ones
                hdst = torch.nn.functional.pad(hdst, (0, (-Dn) % 4))
        else:
            hdst = b.dst_node_feats(pad4=True) if Dn > 0 else None
            if Dn > 0:
                node_src, node_idx = b.src_node_source()
        kp = kspace_width(Dn, De, Dt)
        Wo = self.w_out.weight
        r2 = None
        if Dn > 0:
            # the weights in K-space form, the query bias folded into qt's (qbk), w_out's
            # halves; one kernel each way
            wq_node, wk, wv, qbk, wo1, wo2 = LayerParams.apply(
                self.w_q.weight, self.w_q.bias, self.w_k.weight, self.w_k.bias, self.w_v.weight,
                self.w_v.bias, self.time_enc.w.bias if Dt > 0 else None, Wo, (H, Dn, De, Dt))
            wk, wv = wk.view(H, dh, kp), wv.view(H, dh, kp)
            if hdst.shape[1] > Dn:   # zero-padded rows: the weights take zero columns to match
                wq_node = torch.nn.functional.pad(wq_node, (0, hdst.shape[1] - Dn))
                wo2 = torch.nn.functional.pad(wo2, (0, hdst.shape[1] - Dn))
            # Absorbed keys, head by head: qt[h, v, :] = Q[v, h, :] W_k,aug[h], with
            # q = hdst W_q[:, :Dn]^T and the h_dst half of w_out from one product
            q, r2 = DstProj.apply(hdst, wq_node, wo2)
            qt = HeadProj.apply(q, wk, qbk)
        else:  # one query for every destination: the time part alone (or 1, layers.py:137-140)
            wk = to_kspace(self.w_k.weight, self.w_k.bias, Dn, De, Dt).view(H, dh, kp)
            wv = to_kspace(self.w_v.weight, self.w_v.bias, Dn, De, Dt).view(H, dh, kp)
            wo1 = Wo[:, :D]
            q1 = self._query_bias() if Dt > 0 else torch.ones(D, device=dev)
            qt = HeadProj.apply(q1.view(1, D), wk, None).expand(H, N, kp)

        edge_tab, edge_idx = b.edge_source() if De > 0 else (None, None)
        if node_src is None:
            node_src = torch.empty(E, 0, device=dev)
        if edge_tab is None:
            edge_tab = torch.empty(E, 0, device=dev)
        elif edge_tab.requires_grad:
            raise NotImplementedError("gradients with respect to edge features are not built")
        if Dt > 0:
            tw = self.time_enc.w.weight.view(-1)
            tb = self.time_enc.w.bias
            dt = b.edata["dt"]
        else:
            tw = tb = torch.empty(0, device=dev)
            dt = torch.zeros(E, device=dev)
        split = Dn > 0 and "h" in b.srcdata
        g = _Graph(b.rowptr(), node_idx, edge_tab, edge_idx, dt, N if split else 0)
        link = _TdotLink()
        xbar = TgatAttention.apply(qt, tw, tb, node_src, g, self.negative_slope, drop, drop_seed,
                                   drop_p, link)

        # Absorbed values, head by head: agg[v, h, :] = W_v,aug[h] xbar[h, v, :], then
        # rst = w_out([agg | hdst]) as agg W_o[:, :D]^T + hdst W_o[:, D:]^T + b_o (the
        # bias and the sum in the epilogue kernel).
        agg = HeadReduce.apply(xbar, wv, link)
        r1 = RowsMM.apply(agg, wo1)
        ln = self.layer_norm
        return TgatEpilogue.apply(r1, r2, self.w_out.bias, ln.weight, ln.bias, ln.eps,
                                  out_drop_seed, out_drop_p)


class TGATEncoder(torch.nn.Module):
    """Stack of temporal attention layers fed bottom-up (modules.py:29-35, 48-64): the
    output of layer l becomes ``srcdata['h']`` of the block of layer l+1."""

    def __init__(self, dim_node, dim_edge, dim_time, num_head, dim_out, num_layers=2,
                 dropout=0.1, att_dropout=0.1):
        super().__init__()
        self.layers = torch.nn.ModuleDict()
        self.layers["l0h0"] = TransfomerAttentionLayer(dim_node, dim_edge, dim_time, num_head,
                                                       dropout, att_dropout, dim_out)
        for l in range(1, num_layers):
            self.layers[f"l{l}h0"] = TransfomerAttentionLayer(dim_out, dim_edge, dim_time,
                                                              num_head, dropout, att_dropout,
                                                              dim_out)
        self.num_layers = num_layers

    def forward(self, blocks) -> torch.Tensor:
        rst = None
        for l in range(self.num_layers):
            rst = self.layers[f"l{l}h0"](blocks[l], l, 0)
            if l != self.num_layers - 1:
                blocks[l + 1].srcdata["h"] = rst
        return rst
