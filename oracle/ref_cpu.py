"""CPU restatement of FAST's temporal-attention aggregation path.

TEST INFRASTRUCTURE ONLY. This is the checker the gfx950 kernels are compared against; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. Nothing in ``fast_amd`` uses it.

Two parts:
  * ``C`` - ctypes bindings of ``oracle/fastagg_ref.c``, the scalar restatement of the
    fastAgg operators (getFastAgg/cuda_operators/*), numpy in / numpy out;
  * torch functions restating ``layers.py``'s TGAT layer with DGL semantics
    (``dgl.ops.edge_softmax`` at layers.py:192, ``update_all(copy_u, sum)`` at
    layers.py:207), in float32 or float64, differentiable with torch autograd.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(_HERE, "_build", "liboracle.so")


def build_c(force: bool = False) -> str:
    """Compile the C restatement (gcc, contraction off)."""
    src = os.path.join(_HERE, "fastagg_ref.c")
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(src):
        os.makedirs(os.path.dirname(LIB), exist_ok=True)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
                        "-std=c11", src, "-lm", "-o", LIB], check=True)
    return LIB


class _C:
    def __init__(self):
        self._lib = None

    @property
    def lib(self):
        if self._lib is None:
            self._lib = ctypes.CDLL(build_c())
        return self._lib

    @staticmethod
    def _p(a):
        return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None

    def _call(self, name, *args):
        conv = []
        for a in args:
            if isinstance(a, np.ndarray) or a is None:
                conv.append(self._p(a))
            elif isinstance(a, float):
                conv.append(ctypes.c_float(a))
            else:
                conv.append(ctypes.c_int64(a))
        getattr(self.lib, name)(*conv)

    # --- bookkeeping (bit-exact) ---------------------------------------------------------
    def exclusive_sum(self, x):
        x = np.ascontiguousarray(x, dtype=np.int32)
        out = np.empty(x.size + 1, np.int32)
        self._call("ref_exclusive_sum_i32", x, x.size, out)
        return out

    def cal_deg(self, ids, n_nodes):
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        out = np.empty(n_nodes, np.int32)
        self._call("ref_degree_count_i32", ids, ids.size, out, n_nodes)
        return out

    def balance_mask(self, ptr, threshold):
        ptr = np.ascontiguousarray(ptr, dtype=np.int32)
        out = np.zeros(max(ptr.size - 1, 0), np.int32)
        self.lib.ref_balance_mask_i32(self._p(ptr), ctypes.c_int64(ptr.size),
                                      ctypes.c_int32(threshold), self._p(out))
        return out

    def rowptr(self, dst, n_dst):
        dst = np.ascontiguousarray(dst, dtype=np.int64)
        out = np.empty(n_dst + 1, np.int32)
        self._call("ref_rowptr_from_sorted_dst", dst, dst.size, n_dst, out)
        return out

    # --- softmax -----------------------------------------------------------------------
    def edge_softmax_fwd(self, indptr, x, heads, mode):
        indptr = np.ascontiguousarray(indptr, dtype=np.int32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros((x.shape[0], heads), np.float32)
        self.lib.ref_edge_softmax_fwd_f32(self._p(indptr), ctypes.c_int64(max(indptr.size - 1, 0)),
                                          ctypes.c_int64(x.shape[0]), self._p(x),
                                          ctypes.c_int64(x.shape[1]), ctypes.c_int32(heads),
                                          self._p(y), ctypes.c_int64(heads), ctypes.c_int32(mode))
        return y

    def edge_softmax_bwd(self, indptr, dy, y, heads):
        indptr = np.ascontiguousarray(indptr, dtype=np.int32)
        dy = np.ascontiguousarray(dy, dtype=np.float32)
        y = np.ascontiguousarray(y, dtype=np.float32)
        dx = np.zeros_like(dy)
        self.lib.ref_edge_softmax_bwd_f32(self._p(indptr), ctypes.c_int64(max(indptr.size - 1, 0)),
                                          ctypes.c_int64(dy.shape[0]), self._p(dy),
                                          ctypes.c_int64(dy.shape[1]), self._p(y),
                                          ctypes.c_int64(y.shape[1]), ctypes.c_int32(heads),
                                          self._p(dx), ctypes.c_int64(dx.shape[1]))
        return dx

    def group_softmax_fwd(self, bptr, key, x):
        bptr = np.ascontiguousarray(bptr, dtype=np.int64)
        key = np.ascontiguousarray(key, dtype=np.int64)
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.zeros_like(x)
        self.lib.ref_group_softmax_fwd_f32(self._p(bptr), ctypes.c_int64(key.shape[0]),
                                           self._p(key), ctypes.c_int64(key.shape[1]),
                                           ctypes.c_int64(x.shape[0]), self._p(x),
                                           ctypes.c_int64(x.shape[1]), ctypes.c_int32(x.shape[1]),
                                           self._p(y), ctypes.c_int64(y.shape[1]))
        return y

    def group_softmax_bwd(self, bptr, key, dy, y):
        bptr = np.ascontiguousarray(bptr, dtype=np.int64)
        key = np.ascontiguousarray(key, dtype=np.int64)
        dy = np.ascontiguousarray(dy, dtype=np.float32)
        y = np.ascontiguousarray(y, dtype=np.float32)
        dx = np.zeros_like(dy)
        self.lib.ref_group_softmax_bwd_f32(self._p(bptr), ctypes.c_int64(key.shape[0]),
                                           self._p(key), ctypes.c_int64(key.shape[1]),
                                           ctypes.c_int64(dy.shape[0]), self._p(dy),
                                           ctypes.c_int64(dy.shape[1]), self._p(y),
                                           ctypes.c_int64(y.shape[1]), ctypes.c_int32(dy.shape[1]),
                                           self._p(dx), ctypes.c_int64(dx.shape[1]))
        return dx

    def dropout_mask(self, n_edges, heads, seed, p):
        out = np.empty((n_edges, heads), np.float32)
        self.lib.ref_dropout_mask_f32(ctypes.c_uint64(seed), ctypes.c_float(p),
                                      ctypes.c_int64(n_edges * heads), self._p(out))
        return out

    # --- aggregation -------------------------------------------------------------------
    def edge_scatter_sum(self, dst, src, x, n_out, indptr=None):
        dst = np.ascontiguousarray(dst, dtype=np.int64)
        src = np.ascontiguousarray(src, dtype=np.int64)
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((n_out, x.shape[1]), np.float32)
        ip = None if indptr is None else np.ascontiguousarray(indptr, dtype=np.int32)
        nseg = 0 if ip is None else ip.size - 1
        self.lib.ref_edge_scatter_sum_f32(self._p(dst), self._p(src), ctypes.c_int64(dst.size),
                                          self._p(ip), ctypes.c_int64(nseg), self._p(x),
                                          ctypes.c_int64(x.shape[1]), ctypes.c_int64(x.shape[0]),
                                          ctypes.c_int32(x.shape[1]), self._p(out),
                                          ctypes.c_int64(out.shape[1]), ctypes.c_int64(n_out))
        return out

    def segment_sum(self, indptr, dst, src, x, n_out):
        indptr = np.ascontiguousarray(indptr, dtype=np.int32)
        dst = np.ascontiguousarray(dst, dtype=np.int64)
        src = np.ascontiguousarray(src, dtype=np.int64)
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros((n_out, x.shape[1]), np.float32)
        self.lib.ref_segment_sum_f32(self._p(indptr), ctypes.c_int64(indptr.size - 1), self._p(dst),
                                     self._p(src), ctypes.c_int64(dst.size), self._p(x),
                                     ctypes.c_int64(x.shape[1]), ctypes.c_int64(x.shape[0]),
                                     ctypes.c_int32(x.shape[1]), self._p(out),
                                     ctypes.c_int64(out.shape[1]), ctypes.c_int64(n_out))
        return out

    def fused_attn_fwd(self, indptr, dst, src, n_dst, score, V, slope, p, mask):
        indptr = np.ascontiguousarray(indptr, dtype=np.int32)
        dst = np.ascontiguousarray(dst, dtype=np.int64)
        src = np.ascontiguousarray(src, dtype=np.int64)
        score = np.ascontiguousarray(score, dtype=np.float32)
        V = np.ascontiguousarray(V, dtype=np.float32)
        mask = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
        E, H = score.shape
        dh = V.shape[2]
        attn = np.zeros((E, H), np.float32)
        out = np.zeros((n_dst, H * dh), np.float32)
        self.lib.ref_fused_attn_fwd_f32(self._p(indptr), ctypes.c_int64(indptr.size - 1), self._p(dst),
                                        self._p(src), ctypes.c_int64(E), ctypes.c_int64(n_dst),
                                        self._p(score), self._p(V), ctypes.c_int32(H),
                                        ctypes.c_int32(dh), ctypes.c_float(slope), ctypes.c_float(p),
                                        self._p(mask), self._p(attn), self._p(out))
        return out, attn

    def fused_attn_bwd(self, indptr, dst, src, n_dst, n_src, dout, V, attn, mask, p):
        indptr = np.ascontiguousarray(indptr, dtype=np.int32)
        dst = np.ascontiguousarray(dst, dtype=np.int64)
        src = np.ascontiguousarray(src, dtype=np.int64)
        dout = np.ascontiguousarray(dout, dtype=np.float32)
        V = np.ascontiguousarray(V, dtype=np.float32)
        attn = np.ascontiguousarray(attn, dtype=np.float32)
        mask = None if mask is None else np.ascontiguousarray(mask, dtype=np.float32)
        E, H = attn.shape
        dh = V.shape[2]
        d_act = np.zeros((E, H), np.float32)
        grad_V = np.zeros_like(V)
        self.lib.ref_fused_attn_bwd_f32(self._p(indptr), ctypes.c_int64(indptr.size - 1), self._p(dst),
                                        self._p(src), ctypes.c_int64(E), ctypes.c_int64(n_dst),
                                        ctypes.c_int64(n_src), self._p(dout), self._p(V),
                                        self._p(attn), self._p(mask), ctypes.c_int32(H),
                                        ctypes.c_int32(dh), ctypes.c_float(p), self._p(d_act),
                                        self._p(grad_V))
        return d_act, grad_V


C = _C()


# ---------------------------------------------------------------------------------------
# sampler output -> message-flow-graph blocks (utils.py:67-87) and the sampler's cntE
# ---------------------------------------------------------------------------------------
def sampler_cnte(row) -> np.ndarray:
    """cntE of a sampler result (sampler_core.cpp:384-409, with the leading 0 pushed at
    :247): 0, then the running sum of the lengths of the runs of equal consecutive `row`
    values (the edges grouped by destination). int32."""
    row = np.asarray(row)
    if row.size == 0:
        return np.zeros(1, np.int32)
    ends = np.flatnonzero(np.diff(row) != 0) + 1
    return np.concatenate([[0], ends, [row.size]]).astype(np.int32)


def full_rowptr(row, n_dst: int) -> np.ndarray:
    """The CSR over every destination 0..n_dst of edges sorted by destination `row`
    (zero-degree destinations included): rowptr[v] = number of edges with row < v."""
    return np.searchsorted(np.asarray(row), np.arange(n_dst + 1), side="left").astype(np.int32)


def to_dgl_blocks(ret, hist: int, reverse: bool = False) -> list:
    """utils.py:67-87 without DGL: per sampler result a dict with the edges of
    dgl.create_block((src, dst)) - (col, row) with num_src = dim_in and num_dst = dim_out,
    or (row, col) with the counts swapped when `reverse` - the node ids and timestamps on the
    source side (destination side with `reverse`), dt = dts[dim_out:] (the edges' dts follow
    the dim_out destination entries), the edge ids; grouped `hist` at a time, the incomplete
    last group dropped, the groups reversed."""
    blocks = []
    for r in ret:
        row, col = np.asarray(r.row()).astype(np.int64), np.asarray(r.col()).astype(np.int64)
        dim_in, dim_out = int(r.dim_in()), int(r.dim_out())
        if not reverse:
            b = {"src": col, "dst": row, "num_src": dim_in, "num_dst": dim_out, "node_side": "src"}
        else:
            b = {"src": row, "dst": col, "num_src": dim_out, "num_dst": dim_in, "node_side": "dst"}
        b["ID"] = np.asarray(r.nodes())
        b["ts"] = np.asarray(r.ts())
        b["dt"] = np.asarray(r.dts())[dim_out:]
        b["eID"] = np.asarray(r.eid())
        blocks.append(b)
    groups = [blocks[g * hist:(g + 1) * hist] for g in range(len(blocks) // hist)]
    groups.reverse()
    return groups


# ---------------------------------------------------------------------------------------
# torch restatement of the TGAT layer
# ---------------------------------------------------------------------------------------
def time_encoding_weight(dim: int) -> torch.Tensor:
    """w = 1/10**linspace(0, 9, dim) in float32 (layers.py:14)."""
    return torch.from_numpy(1 / 10 ** np.linspace(0, 9, dim, dtype=np.float32))


def time_encode(dt: torch.Tensor, w: torch.Tensor, b: torch.Tensor, dtype=torch.float64):
    """cos(w*t + b) (layers.py:17-29). The argument is the float32 value of the reference's
    Linear(1, Dt) (rounded product, then rounded sum); the cosine and everything after it
    are evaluated in ``dtype``. Differentiable in w and b."""
    t = dt.to(torch.float32).reshape(-1, 1)
    arg32 = (t * w.to(torch.float32).reshape(1, -1)) + b.to(torch.float32).reshape(1, -1)
    if dtype == torch.float32:
        return torch.cos(arg32)
    # Same forward value as cos(arg32) evaluated in dtype; gradients of the exact
    # expression in dtype.
    arg = t.to(dtype) * w.to(dtype).reshape(1, -1) + b.to(dtype).reshape(1, -1)
    arg = arg + (arg32.to(dtype) - arg).detach()
    return torch.cos(arg)


def edge_softmax(scores: torch.Tensor, dst: torch.Tensor, num_dst: int) -> torch.Tensor:
    """Softmax over the incoming edges of every destination (dgl.ops.edge_softmax,
    layers.py:192): exp(x - max) / sum per destination and head."""
    H = scores.shape[1]
    idx = dst.view(-1, 1).expand(-1, H)
    mx = torch.full((num_dst, H), -float("inf"), dtype=scores.dtype)
    mx = mx.scatter_reduce(0, idx, scores, reduce="amax", include_self=True)
    ex = torch.exp(scores - mx[dst].detach())
    den = torch.zeros((num_dst, H), dtype=scores.dtype).index_add(0, dst, ex)
    return ex / den[dst]


def copy_u_sum(v_src: torch.Tensor, src: torch.Tensor, dst: torch.Tensor, num_dst: int):
    """update_all(copy_u('v','m'), sum('m','h')) (layers.py:207): out[d] = sum of source
    rows over the incoming edges; zero-degree destinations get 0."""
    out = torch.zeros((num_dst, v_src.shape[1]), dtype=v_src.dtype)
    return out.index_add(0, dst, v_src[src])


def layer_params(layer) -> dict:
    """CPU float64 copies (leaf tensors) of a TransfomerAttentionLayer's parameters."""
    out = {}
    for name, p in layer.named_parameters():
        out[name] = p.detach().to("cpu", torch.float64).clone().requires_grad_(True)
    out["_eps"] = layer.layer_norm.eps
    out["_heads"] = layer.num_head
    out["_dims"] = (layer.dim_node_feat, layer.dim_edge_feat, layer.dim_time, layer.dim_out)
    return out


# Half-width of the kink bands, relative to the absolute terms of the pre-activation value.
KINK_RTOL = 1e-5


def _kink(name, z, zabs, hint, slope, stats):
    """The branch (z > 0) of a piecewise-linear activation, with an implementation's branch
    taken inside the band |z| <= KINK_RTOL * zabs around the kink. ``hint`` holds the
    implementation's post-activation values (their signs are its branches; slope > 0 maps
    them back to its pre-activation values, which give the deviation statistics)."""
    with torch.no_grad():
        near = z.abs() <= KINK_RTOL * zabs
        mine = hint > 0
        pos = torch.where(near, mine, z > 0)
        if stats is not None:
            pre = torch.where(mine, hint, hint / slope) if slope > 0 else hint
            seen = mine if slope <= 0 else torch.ones_like(mine)
            dev = ((pre.to(z.dtype) - z).abs() / zabs.clamp_min(1e-300))[seen & (zabs > 0)]
            zero = zabs == 0   # exactly at the kink: every term is 0 (a dropped entry)
            stats[name + "_zero"] = stats.get(name + "_zero", 0) + int(zero.sum())
            stats[name + "_near"] = stats.get(name + "_near", 0) + int((near & ~zero).sum())
            stats[name + "_disagree"] = (stats.get(name + "_disagree", 0)
                                         + int((mine != (z > 0))[~near].sum()))
            stats[name + "_dev"] = max(stats.get(name + "_dev", 0.0),
                                       float(dev.max()) if dev.numel() else 0.0)
    return pos


def tgat_layer(P: dict, h: torch.Tensor, f: torch.Tensor, dt: torch.Tensor, src: torch.Tensor,
               dst: torch.Tensor, num_dst: int, slope: float = 0.2, att_drop=None,
               dtype=torch.float64, out_drop=None, hints=None, kink_stats=None) -> torch.Tensor:
    """layers.py:98-240, TGAT branch with DGL semantics, eval-mode dropout except for an
    optional attention multiplier ``att_drop`` [E,H] and an optional output multiplier
    ``out_drop`` [N,D] (keep/(1-p) or 0).

    h: [N+E, Dn] source-node features (row N+e feeds edge e); f: [E, De]; dt: [E];
    src/dst: int64 [E] source / destination ids.

    ``hints`` (optional dict): an implementation's post-activation values, "score" [E,H]
    (after LeakyReLU) and "relu" [N,D] (after the output dropout and ReLU). LeakyReLU's and
    ReLU's derivatives jump at 0, so for a pre-activation value within float32 rounding of 0
    the branch is not fixed by the inputs at float32 precision: where |z| <= KINK_RTOL times
    the sum of the absolute values of z's terms, the restatement takes the implementation's
    branch (the sign of its value); everywhere else the sign of its own z. With a dict
    ``kink_stats`` it adds, per activation ("score", "relu"), the entries in the band
    ("_near", not counting those whose terms are all 0, "_zero"), the entries outside it
    whose hinted branch differs from the sign of z ("_disagree"), and keeps the largest
    deviation of the implementation's pre-activation value from z, relative to the absolute
    terms ("_dev"; for ReLU over the entries the implementation kept).
    """
    Dn, De, Dt, D = P["_dims"]
    H = P["_heads"]
    N, E = num_dst, dst.numel()
    if E == 0:  # layers.py:101-102
        return torch.zeros((N, D), dtype=dtype)
    cast = lambda t: t.to(dtype)
    hq = [cast(h[:N])] if Dn else []
    hk = [cast(h[N:])] if Dn else []
    if De:
        hk.append(cast(f))
    if Dt:
        tw, tb = P["time_enc.w.weight"].view(-1), P["time_enc.w.bias"]
        hk.append(time_encode(dt, tw, tb, dtype))
        hq.append(time_encode(torch.zeros(N), tw, tb, dtype))
    if Dn + Dt > 0:
        Q = torch.nn.functional.linear(torch.cat(hq, 1), cast(P["w_q.weight"]), cast(P["w_q.bias"]))
    else:
        Q = torch.ones((N, D), dtype=dtype)
    kv = torch.cat(hk, 1)
    Q = Q[dst]
    K = torch.nn.functional.linear(kv, cast(P["w_k.weight"]), cast(P["w_k.bias"]))
    V = torch.nn.functional.linear(kv, cast(P["w_v.weight"]), cast(P["w_v.bias"]))
    Q, K, V = Q.view(E, H, -1), K.view(E, H, -1), V.view(E, H, -1)
    z = (Q * K).sum(2)
    if hints is None or "score" not in hints:
        scores = torch.nn.functional.leaky_relu(z, slope)
    else:
        with torch.no_grad():
            kabs = torch.nn.functional.linear(kv.abs(), cast(P["w_k.weight"]).abs(),
                                              cast(P["w_k.bias"]).abs()).view(E, H, -1)
            zabs = (Q.abs() * kabs).sum(2)
        pos = _kink("score", z, zabs, hints["score"], slope, kink_stats)
        scores = torch.where(pos, z, slope * z)
    att = edge_softmax(scores, dst, N)
    if att_drop is not None:
        att = att * cast(att_drop)
    v = (V * att[:, :, None]).reshape(E, -1)
    v_src = torch.cat([torch.zeros((N, v.shape[1]), dtype=dtype), v], 0)
    agg = copy_u_sum(v_src, src, dst, N)
    rst = torch.cat([agg, cast(h[:N])], 1) if Dn else agg
    rin = rst
    rst = torch.nn.functional.linear(rin, cast(P["w_out.weight"]), cast(P["w_out.bias"]))
    if out_drop is not None:  # layers.py:235 self.dropout, as multipliers [N, D]
        rst = rst * cast(out_drop)
    if hints is None or "relu" not in hints:
        rst = torch.relu(rst)
    else:
        with torch.no_grad():
            uabs = torch.nn.functional.linear(rin.abs(), cast(P["w_out.weight"]).abs(),
                                              cast(P["w_out.bias"]).abs())
            if out_drop is not None:
                uabs = uabs * cast(out_drop)
        pos = _kink("relu", rst, uabs, hints["relu"], 0.0, kink_stats)
        rst = torch.where(pos, rst, torch.zeros_like(rst))
    return torch.nn.functional.layer_norm(rst, (D,), cast(P["layer_norm.weight"]),
                                          cast(P["layer_norm.bias"]), P["_eps"])
