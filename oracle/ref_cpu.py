"""CPU restatement of FAST's temporal-attention aggregation path.

TEST INFRASTRUCTURE ONLY. This is the checker the gfx950 kernels are compared against; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. Nothing in ``fast_amd`` uses it.

Two parts:
  * ``C`` - ctypes bindings of ``oracle/fastagg_ref.c``, the scalar restatement of the
    fastAgg operators (getFastAgg/cuda_operators/*), numpy in / numpy out;
  * torch functions restating ``layers.py``'s TGAT layer with DGL semantics
    (``dgl.ops.edge_softmax`` at layers.py:192, ``update_all(copy_u, sum)`` at
    layers.py:207), in float32 or float64, differentiable with torch autograd;
  * the TGN node memory of ``memorys.py`` (mail gather, GRU / RNN updater, the mailbox and
    memory write-back), numpy state, torch for the differentiable updater.
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



# ---------------------------------------------------------------------------------------
# TGN node memory (memorys.py)
# ---------------------------------------------------------------------------------------
def mailbox_state(num_nodes: int, m: int, de: int, slots: int, seed: int = 0) -> dict:
    """A MailBox's tensors (memorys.py:13-18) as numpy arrays, filled with seeded values."""
    rng = np.random.default_rng(seed)
    return {"node_memory": rng.standard_normal((num_nodes, m)).astype(np.float32),
            "node_memory_ts": (rng.random(num_nodes) * 1e5).astype(np.float32),
            "mailbox": rng.standard_normal((num_nodes, slots, 2 * m + de)).astype(np.float32),
            "mailbox_ts": (rng.random((num_nodes, slots)) * 1e5).astype(np.float32),
            "next_mail_pos": rng.integers(0, slots, num_nodes).astype(np.int64)}


def mail_inputs(state: dict, ids) -> dict:
    """MailBox.prep_input_mails (memorys.py:67-71): per source row its node's memory, memory
    time, mails (flattened over the slots) and mail times. Ids outside [0, num_nodes) give
    zero rows (the reference raises; this is the convention of the GPU path)."""
    ids = np.asarray(ids, dtype=np.int64)
    n_nodes = state["node_memory"].shape[0]
    ok = (ids >= 0) & (ids < n_nodes)
    safe = np.where(ok, ids, 0)

    def take(a):
        out = a[safe].copy()
        out[~ok] = 0
        return out

    mb = state["mailbox"]
    return {"mem": take(state["node_memory"]), "mem_ts": take(state["node_memory_ts"]),
            "mem_input": take(mb.reshape(mb.shape[0], -1)), "mail_ts": take(state["mailbox_ts"])}


def recurrent_update(P: dict, mem_input, mem, ts, mem_ts, gru: bool = True,
                     dtype=torch.float64) -> torch.Tensor:
    """GRUMemeoryUpdater / RNNMemeoryUpdater.forward (memorys.py:286-293, 322-329) in
    ``dtype``: the time features of ts - mem_ts (a float32 difference, as in the reference)
    by ``time_encode``; x = [mem_input, time features]; then torch.nn.GRUCell's equations
    with gate blocks (r, z, n) - r = s(gi_r + gh_r), z = s(gi_z + gh_z),
    n = tanh(gi_n + r gh_n), h' = (1 - z) n + z h - or RNNCell's h' = tanh(gi + gh), where
    gi = x W_ih^T + b_ih and gh = h W_hh^T + b_hh. P holds 'updater.weight_ih',
    'updater.weight_hh', 'updater.bias_ih', 'updater.bias_hh' and, with time features,
    'time_enc.w.weight' / 'time_enc.w.bias'. Differentiable in every P entry and in mem."""
    cast = lambda t: torch.as_tensor(t).to(dtype)
    x = cast(mem_input)
    if "time_enc.w.weight" in P:
        t = torch.as_tensor(ts).to(torch.float32) - torch.as_tensor(mem_ts).to(torch.float32)
        tf = time_encode(t, P["time_enc.w.weight"].view(-1), P["time_enc.w.bias"], dtype)
        x = torch.cat([x, tf], dim=1)
    h = cast(mem)
    gi = x @ cast(P["updater.weight_ih"]).t() + cast(P["updater.bias_ih"])
    gh = h @ cast(P["updater.weight_hh"]).t() + cast(P["updater.bias_hh"])
    if not gru:
        return torch.tanh(gi + gh)
    m = h.shape[1]
    r = torch.sigmoid(gi[:, :m] + gh[:, :m])
    z = torch.sigmoid(gi[:, m:2 * m] + gh[:, m:2 * m])
    n = torch.tanh(gi[:, 2 * m:] + r * gh[:, 2 * m:])
    return (1 - z) * n + z * h


def combine_node_feature(P: dict, h, updated, dim_node_feat: int, dim_hid: int,
                         dtype=torch.float64):
    """memorys.py:297-304: the updated memory added to, mapped onto, or in place of the
    node features."""
    if dim_node_feat > 0:
        if dim_node_feat == dim_hid:
            return torch.as_tensor(h).to(dtype) + updated
        return updated + (torch.as_tensor(h).to(dtype) @ P["node_feat_map.weight"].to(dtype).t()
                          + P["node_feat_map.bias"].to(dtype))
    return updated


def _last_rows(ids: np.ndarray) -> np.ndarray:
    """Row of the last occurrence of every distinct id (ascending ids)."""
    rev = ids[::-1]
    _, first = np.unique(rev, return_index=True)
    return len(ids) - 1 - first


def update_memory(state: dict, nid, memory, ts, root_count: int, neg_samples: int = 1) -> None:
    """MailBox.update_memory (memorys.py:86-103): node_memory / node_memory_ts of the first
    2n rows (n = root_count // (neg_samples + 2)), the last row of a repeated id winning (the
    reference's device index_put leaves that winner unspecified)."""
    k = root_count // (neg_samples + 2) * 2
    nid = np.asarray(nid, dtype=np.int64)[:k]
    memory = np.asarray(memory, dtype=np.float32)[:k]
    ts = np.asarray(ts, dtype=np.float32)[:k]
    rows = _last_rows(nid)
    ok = (nid[rows] >= 0) & (nid[rows] < state["node_memory"].shape[0])
    rows = rows[ok]
    state["node_memory"][nid[rows]] = memory[rows]
    state["node_memory_ts"][nid[rows]] = ts[rows]


def update_mailbox(state: dict, memory, root_nodes, ts, edge_feats, neg_samples: int = 1) -> None:
    """MailBox.update_mailbox for deliver_to 'self', mail_combine 'last' (memorys.py:113-139):
    for the n = len(root_nodes) // (neg_samples + 2) true edges, source mail
    [mem_src, mem_dst, ef] and destination mail [mem_dst, mem_src, ef], interleaved
    (cat(dim=1).reshape); the interleaved row r is paired with ts[r]; unique node ids with
    the last row of each (torch.unique + scatter_ of arange); slot next_mail_pos written and,
    with more than one slot, advanced modulo the slot count."""
    n = len(root_nodes) // (neg_samples + 2)
    roots = np.asarray(root_nodes, dtype=np.int64)
    memory = np.asarray(memory, dtype=np.float32)
    mem_src, mem_dst = memory[:n], memory[n:2 * n]
    parts_s, parts_d = [mem_src, mem_dst], [mem_dst, mem_src]
    if edge_feats is not None and np.asarray(edge_feats).size:
        ef = np.asarray(edge_feats, dtype=np.float32)[:n]
        parts_s.append(ef)
        parts_d.append(ef)
    src_mail = np.concatenate(parts_s, axis=1)
    dst_mail = np.concatenate(parts_d, axis=1)
    mail = np.concatenate([src_mail, dst_mail], axis=1).reshape(2 * n, -1)
    nid = np.stack([roots[:n], roots[n:2 * n]], axis=1).reshape(-1)
    mail_ts = np.asarray(ts, dtype=np.float32)[:2 * n]
    perm = _last_rows(nid)
    nid, mail, mail_ts = nid[perm], mail[perm], mail_ts[perm]
    ok = (nid >= 0) & (nid < state["mailbox"].shape[0])
    nid, mail, mail_ts = nid[ok], mail[ok], mail_ts[ok]
    slots = state["mailbox"].shape[1]
    pos = state["next_mail_pos"][nid]
    state["mailbox"][nid, pos] = mail
    state["mailbox_ts"][nid, pos] = mail_ts
    if slots > 1:
        state["next_mail_pos"][nid] = (pos + 1) % slots
