"""The CPU restatement (oracle/) pinned on the CPU, no GPU needed.

Three kinds of checks, chosen so that an index, sign, operand-order or concatenation-order
mistake in the oracle fails at least one of them:
  * the golden fixtures under tests/golden/ (plain-Python loops over the definitions,
    written by tests/golden/make_golden.py without touching oracle/);
  * closed forms and invariants of the operations (softmax sums to 1 and is shift
    invariant, degree-1 segments give exactly 1, scatter-sum is the adjoint of the gather,
    a one-key batched softmax is the segment softmax, ...);
  * finite differences of the layer (fixture) against the oracle's autograd gradients.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import ref_cpu
from oracle.ref_cpu import C
from tests._util import FP32_TOL, assert_rel, rel_err

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with open(os.path.join(GOLD, name)) as fh:
        return json.load(fh)


def _csr_from_degrees(degs):
    """indptr over the non-empty segments and the dst id of every edge."""
    dst = np.repeat(np.arange(len(degs)), degs).astype(np.int64)
    nz = np.asarray([d for d in degs if d > 0], dtype=np.int64)
    indptr = np.concatenate([[0], np.cumsum(nz)]).astype(np.int32)
    return indptr, dst


# ---------------------------------------------------------------------------------------
# bookkeeping: bit-exact integers
# ---------------------------------------------------------------------------------------
def test_bookkeeping_golden():
    g = _load("bookkeeping.json")
    for c in g["exclusive_sum"]:
        np.testing.assert_array_equal(C.exclusive_sum(np.asarray(c["in"], np.int64)), c["out"])
    for c in g["cal_deg"]:
        np.testing.assert_array_equal(C.cal_deg(np.asarray(c["ids"], np.int64), c["n_nodes"]),
                                      c["out"])
    for c in g["balance_mask"]:
        np.testing.assert_array_equal(C.balance_mask(np.asarray(c["ptr"]), c["threshold"]),
                                      c["out"])
    for c in g["rowptr"]:
        np.testing.assert_array_equal(C.rowptr(np.asarray(c["dst"], np.int64), c["n_dst"]),
                                      c["out"])


def test_cnte_golden():
    """The sampler's cntE (run lengths of the sorted row array, cumulated) is the exclusive
    sum of the per-destination counts of the non-empty destinations (unique2indptr)."""
    for c in _load("bookkeeping.json")["cnte"]:
        dst = np.asarray(c["dst"], np.int64)
        _, counts = np.unique(dst, return_counts=True)
        np.testing.assert_array_equal(C.exclusive_sum(counts), c["out"])


class _GoldenSample:
    """A sampler result with the FAST sampler's accessors, from a golden fixture entry."""

    def __init__(self, d):
        self.d = d

    def row(self): return np.asarray(self.d["row"], np.int32)
    def col(self): return np.asarray(self.d["col"], np.int32)
    def nodes(self): return np.asarray(self.d["nodes"], np.int64)
    def dts(self): return np.asarray(self.d["dts"], np.float32)
    def ts(self): return np.asarray(self.d["ts"], np.float32)
    def eid(self): return np.asarray(self.d["eid"], np.int64)
    def dim_in(self): return self.d["dim_in"]
    def dim_out(self): return self.d["dim_out"]


def test_to_dgl_blocks_golden():
    """oracle.to_dgl_blocks (utils.py:67-87) against the blocks of the golden fixture, for
    hist 1 and 2 (an odd result count: the incomplete last group is dropped) and both
    directions; the sampler's cntE and the full CSR likewise."""
    c = _load("mfg.json")
    ret = [_GoldenSample(d) for d in c["results"]]
    for key, want in c["blocks"].items():
        hist, rev = int(key[4]), key.endswith("rev1")
        got = ref_cpu.to_dgl_blocks(ret, hist, reverse=rev)
        assert [len(g) for g in got] == [len(g) for g in want], key
        for gg, gw in zip(got, want):
            for b, w in zip(gg, gw):
                for k in ("num_src", "num_dst", "node_side"):
                    assert b[k] == w[k], (key, k)
                for k in ("src", "dst", "ID", "eID"):
                    np.testing.assert_array_equal(b[k], np.asarray(w[k]), err_msg=f"{key} {k}")
                for k in ("ts", "dt"):
                    np.testing.assert_array_equal(b[k], np.asarray(w[k], np.float32), err_msg=f"{key} {k}")
    for r, cn, rp in zip(ret, c["cnte"], c["rowptr"]):
        np.testing.assert_array_equal(ref_cpu.sampler_cnte(r.row()), cn)
        np.testing.assert_array_equal(ref_cpu.full_rowptr(r.row(), r.dim_out()), rp)
        np.testing.assert_array_equal(C.rowptr(r.row(), r.dim_out()), rp)


def test_bookkeeping_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.integers(0, 50, 10_000)
    np.testing.assert_array_equal(C.exclusive_sum(x), np.concatenate([[0], np.cumsum(x)]))
    ids = rng.integers(-3, 700, 20_000)
    ref = np.bincount(ids[(ids >= 0) & (ids < 650)], minlength=650)
    np.testing.assert_array_equal(C.cal_deg(ids, 650), ref)
    degs = rng.integers(0, 6, 500)
    dst = np.repeat(np.arange(500), degs)
    np.testing.assert_array_equal(C.rowptr(dst, 500), np.concatenate([[0], np.cumsum(degs)]))
    # threshold 1 on a strictly increasing pointer marks every non-empty entry
    ptr = np.concatenate([[0], np.cumsum(rng.integers(1, 4, 300))])
    np.testing.assert_array_equal(C.balance_mask(ptr, 1), np.ones(300, np.int32))


# ---------------------------------------------------------------------------------------
# segment softmax (edge_softmax.cu:255-329 formula; dgl.ops.edge_softmax semantics)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("mode", [0, 1])
def test_edge_softmax_golden(mode):
    for c in _load("softmax.json"):
        x = np.asarray(c["x"], np.float32)
        y = C.edge_softmax_fwd(c["indptr"], x, c["heads"], mode)
        assert_rel(y, c["y"], FP32_TOL, f"softmax mode {mode}")
        dx = C.edge_softmax_bwd(c["indptr"], np.asarray(c["dy"], np.float32), y, c["heads"])
        assert_rel(dx, c["dx"], FP32_TOL, "softmax backward")


def test_torch_edge_softmax_golden():
    """The float64 torch restatement used inside the layer oracle, forward and autograd."""
    for c in _load("softmax.json"):
        ip = np.asarray(c["indptr"])
        dst = torch.from_numpy(np.repeat(np.arange(ip.size - 1), np.diff(ip)))
        x = torch.tensor(c["x"], dtype=torch.float64, requires_grad=True)
        y = ref_cpu.edge_softmax(x, dst, ip.size - 1)
        assert rel_err(y, c["y"]) < 1e-12
        y.backward(torch.tensor(c["dy"], dtype=torch.float64))
        assert rel_err(x.grad, c["dx"]) < 1e-12


def test_edge_softmax_invariants():
    rng = np.random.default_rng(11)
    degs = [1, 2, 7, 64, 65, 300, 1, 3]
    indptr, dst = _csr_from_degrees(degs)
    E, H = dst.size, 3
    x = (rng.standard_normal((E, H)) * 4).astype(np.float32)
    y = C.edge_softmax_fwd(indptr, x, H, 0)
    seg_sum = np.add.reduceat(y.astype(np.float64), indptr[:-1], axis=0)
    np.testing.assert_allclose(seg_sum, 1.0, rtol=0, atol=1e-5)
    # degree-1 segments give exactly 1
    for s, d in enumerate([d for d in degs if d]):
        if d == 1:
            assert np.all(y[indptr[s]] == 1.0)
    # shift invariance within a segment (shift by a per-segment constant)
    shift = np.repeat(rng.uniform(-20, 20, len(degs)), degs).astype(np.float32)[:, None]
    y2 = C.edge_softmax_fwd(indptr, (x.astype(np.float64) + shift).astype(np.float32), H, 0)
    assert rel_err(y2, y) < 1e-4  # the shifted inputs are re-rounded to float32
    # equal scores in a segment give 1/deg
    yeq = C.edge_softmax_fwd(indptr, np.ones_like(x), H, 1)
    ref = np.repeat(1.0 / np.asarray(degs, np.float64), degs)[:, None] * np.ones((1, H))
    assert rel_err(yeq, ref) < 1e-6
    # the backward is orthogonal to the constants: its per-segment sum vanishes
    dy = rng.standard_normal((E, H)).astype(np.float32)
    dx = C.edge_softmax_bwd(indptr, dy, y, H)
    np.testing.assert_allclose(np.add.reduceat(dx.astype(np.float64), indptr[:-1], axis=0), 0.0,
                               atol=1e-5)


def test_group_softmax_reduces_to_segment_softmax():
    """One key per batch: the batched softmax is the segment softmax of the batches. With two
    interleaved keys it is the segment softmax of the edges sorted by (batch, key)."""
    rng = np.random.default_rng(5)
    degs = [3, 9, 1, 12]
    bptr = np.concatenate([[0], np.cumsum(degs)]).astype(np.int64)
    E, L = int(bptr[-1]), max(degs)
    x = rng.standard_normal((E, 2)).astype(np.float32)
    dy = rng.standard_normal((E, 2)).astype(np.float32)
    key0 = np.zeros((len(degs), L), np.int64)
    y = C.group_softmax_fwd(bptr, key0, x)
    y_ref = C.edge_softmax_fwd(bptr.astype(np.int32), x, 2, 1)
    assert rel_err(y, y_ref) < 1e-6
    assert rel_err(C.group_softmax_bwd(bptr, key0, dy, y),
                   C.edge_softmax_bwd(bptr.astype(np.int32), dy, y_ref, 2)) < 1e-6
    # interleaved keys 0/1 inside every batch
    key = np.zeros((len(degs), L), np.int64)
    for b, d in enumerate(degs):
        key[b, :d] = np.arange(d) % 2
    y = C.group_softmax_fwd(bptr, key, x)
    order, seg = [], [0]
    for b, d in enumerate(degs):
        for k in (0, 1):
            idx = [bptr[b] + j for j in range(d) if key[b, j] == k]
            if idx:
                order += idx
                seg.append(seg[-1] + len(idx))
    order = np.asarray(order)
    ys = C.edge_softmax_fwd(np.asarray(seg, np.int32), x[order], 2, 1)
    assert rel_err(y[order], ys) < 1e-6


# ---------------------------------------------------------------------------------------
# aggregation (update_all(copy_u, sum) semantics; aggregate_*.cu)
# ---------------------------------------------------------------------------------------
def test_aggregation_golden():
    for c in _load("aggregation.json"):
        dst, src = np.asarray(c["dst"], np.int64), np.asarray(c["src"], np.int64)
        x = np.asarray(c["x"], np.float32)
        N = c["n_dst"]
        assert_rel(C.edge_scatter_sum(dst, src, x, N), c["agg"], FP32_TOL, "scatter sum")
        assert_rel(C.segment_sum(c["indptr"], dst, src, x, N), c["agg"], FP32_TOL, "segment sum")
        # backward = scatter of dout[dst] into the source rows
        dx = C.edge_scatter_sum(src, dst, np.asarray(c["dout"], np.float32), x.shape[0])
        assert_rel(dx, c["dx"], FP32_TOL, "scatter-sum backward")
        got = ref_cpu.copy_u_sum(torch.from_numpy(x).double(), torch.from_numpy(src),
                                 torch.from_numpy(dst), N)
        assert rel_err(got, c["agg"]) < 1e-12


def test_aggregation_adjoint():
    """<A x, y> == <x, A^T y> for the gather-sum A and its transpose; empty dst rows are 0."""
    rng = np.random.default_rng(8)
    degs = [0, 4, 1, 0, 9, 2]
    indptr, dst = _csr_from_degrees(degs)
    N, E, dim = len(degs), dst.size, 5
    src = rng.permutation(np.arange(N, N + E)).astype(np.int64)
    x = rng.standard_normal((N + E, dim)).astype(np.float32)
    yv = rng.standard_normal((N, dim)).astype(np.float32)
    ax = C.edge_scatter_sum(dst, src, x, N)
    aty = C.edge_scatter_sum(src, dst, yv, N + E)
    assert math.isclose(float((ax.astype(np.float64) * yv).sum()),
                        float((x.astype(np.float64) * aty).sum()), rel_tol=1e-5)
    assert np.all(ax[[0, 3]] == 0.0)
    assert_rel(C.segment_sum(indptr, dst, src, x, N), ax, FP32_TOL, "segment vs scatter")


# ---------------------------------------------------------------------------------------
# fused LeakyReLU + softmax + dropout + aggregation (fused_attention.cu intended semantics)
# ---------------------------------------------------------------------------------------
def test_fused_attn_golden():
    c = _load("fused_attn.json")
    dst, src = np.asarray(c["dst"], np.int64), np.asarray(c["src"], np.int64)
    score, V = np.asarray(c["score"], np.float32), np.asarray(c["V"], np.float32)
    mask = np.asarray(c["mask"], np.float32)
    N = c["n_dst"]
    out, attn = C.fused_attn_fwd(c["indptr"], dst, src, N, score, V, c["slope"], c["p"], mask)
    assert_rel(attn, c["attn"], FP32_TOL, "fused attn")
    assert_rel(out, c["out"], FP32_TOL, "fused out")
    d_act, gV = C.fused_attn_bwd(c["indptr"], dst, src, N, N + dst.size,
                                 np.asarray(c["dout"], np.float32), V, attn, mask, c["p"])
    assert_rel(d_act, c["d_act"], FP32_TOL, "fused d_act")
    assert_rel(gV, c["grad_V"], FP32_TOL, "fused grad_V")


# ---------------------------------------------------------------------------------------
# time encoding (layers.py:10-29)
# ---------------------------------------------------------------------------------------
def test_time_weight_golden():
    g = _load("time_weight.json")
    w = ref_cpu.time_encoding_weight(100).numpy()
    np.testing.assert_array_equal(w, np.asarray(g["w_float32"], np.float32))
    # float32 exponents up to 9 carry a relative error of up to 9 * ln(10) * 2^-24 ~ 1.2e-6
    np.testing.assert_allclose(w.astype(np.float64), g["w_exact"], rtol=1.5e-6)


def test_time_encode_closed_form():
    w = ref_cpu.time_encoding_weight(7).double().requires_grad_(True)
    b = torch.linspace(-1.0, 2.0, 7, dtype=torch.float64).requires_grad_(True)
    # dt = 0 gives cos(b); with b = 0 exactly 1
    assert torch.equal(ref_cpu.time_encode(torch.zeros(3), w.detach(), torch.zeros(7)),
                       torch.ones(3, 7, dtype=torch.float64))
    z = ref_cpu.time_encode(torch.zeros(2), w, b)
    assert rel_err(z, torch.cos(b.detach()).expand(2, 7)) < 1e-7
    # the argument is the float32 Linear(1, Dt) value: rounded product, then rounded sum
    t = torch.tensor([0.0, 3.5, 1234.0, 9.0e5])
    t32, w32, b32 = t.numpy()[:, None], w.detach().float().numpy()[None], b.detach().float().numpy()[None]
    arg = torch.from_numpy(((t32 * w32).astype(np.float32) + b32).astype(np.float32)).double()
    y = ref_cpu.time_encode(t, w, b)
    assert rel_err(y, torch.cos(arg)) < 1e-15
    # gradients at that point: d/dw = -sin(arg) * t, d/db = -sin(arg)
    gy = torch.randn(4, 7, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    y.backward(gy)
    sn = torch.sin(arg)
    assert rel_err(w.grad, (-sn * t.double()[:, None] * gy).sum(0)) < 1e-6
    assert rel_err(b.grad, (-sn * gy).sum(0)) < 1e-6


# ---------------------------------------------------------------------------------------
# one TGAT layer (layers.py:98-240, TGAT branch) against plain loops + finite differences
# ---------------------------------------------------------------------------------------
def _layer_case():
    c = _load("tgat_layer_tiny.json")
    Dn, De, Dt, H, D = c["dims"]
    T = lambda v: torch.tensor(v, dtype=torch.float64)
    P = {
        "time_enc.w.weight": T(c["P"]["tw"]).view(-1, 1), "time_enc.w.bias": T(c["P"]["tb"]),
        "w_q.weight": T(c["P"]["Wq"]), "w_q.bias": T(c["P"]["bq"]),
        "w_k.weight": T(c["P"]["Wk"]), "w_k.bias": T(c["P"]["bk"]),
        "w_v.weight": T(c["P"]["Wv"]), "w_v.bias": T(c["P"]["bv"]),
        "w_out.weight": T(c["P"]["Wo"]), "w_out.bias": T(c["P"]["bo"]),
        "layer_norm.weight": T(c["P"]["lnw"]), "layer_norm.bias": T(c["P"]["lnb"]),
    }
    for v in P.values():
        v.requires_grad_(True)
    P.update({"_eps": 1e-5, "_heads": H, "_dims": (Dn, De, Dt, D)})
    N = len(c["degs"])
    dst = torch.tensor(c["dst"], dtype=torch.int64)
    src = torch.arange(N, N + dst.numel())
    h = T(c["h"]).requires_grad_(True)
    return c, P, h, src, dst, N


def test_tgat_layer_golden_forward():
    c, P, h, src, dst, N = _layer_case()
    out = ref_cpu.tgat_layer(P, h, torch.tensor(c["f"]), torch.tensor(c["dt"], dtype=torch.float32),
                             src, dst, N)
    assert rel_err(out, c["out"]) < 1e-10


def test_tgat_layer_golden_gradients():
    c, P, h, src, dst, N = _layer_case()
    out = ref_cpu.tgat_layer(P, h, torch.tensor(c["f"]), torch.tensor(c["dt"], dtype=torch.float32),
                             src, dst, N)
    (out * torch.tensor(c["wsum"], dtype=torch.float64)).sum().backward()
    names = {"Wk": "w_k.weight", "Wv": "w_v.weight", "Wq": "w_q.weight", "tb": "time_enc.w.bias",
             "tw": "time_enc.w.weight", "Wo": "w_out.weight", "bk": "w_k.bias"}
    for key, fd in c["fd_grads"].items():
        name, idx = key.split("[")
        idx = [int(i) for i in idx.rstrip("]").split(",")]
        grad = h.grad if name == "h" else P[names[name]].grad
        got = float(grad[tuple(idx)] if len(idx) > 1 or name != "tw" else grad[idx[0], 0])
        # The differences were taken with the exact time argument, the oracle rounds it to
        # float32 like the reference (|arg| ~ 1e4, so cos moves by up to ~5e-4 relative).
        assert math.isclose(got, fd, rel_tol=5e-4, abs_tol=1e-6), (key, got, fd)


def _grads_with_hints(c, P, h, src, dst, N, hints, stats=None):
    for v in list(P.values()) + [h]:
        if isinstance(v, torch.Tensor) and v.grad is not None:
            v.grad = None
    out = ref_cpu.tgat_layer(P, h, torch.tensor(c["f"]), torch.tensor(c["dt"], dtype=torch.float32),
                             src, dst, N, hints=hints, kink_stats=stats)
    (out * torch.tensor(c["wsum"], dtype=torch.float64)).sum().backward()
    return out.detach(), {k: v.grad.clone() for k, v in P.items()
                          if isinstance(v, torch.Tensor) and v.grad is not None}


def test_tgat_layer_branch_hints_outside_the_kink_band_change_nothing():
    """With branch hints, the restatement takes them only inside the float32 rounding band of
    a kink: hints of either sign everywhere (every score of this case is far from 0) give the
    plain layer, and the hinted branches outside the band are counted as disagreeing where
    they differ from the sign of z (all of them, over the two hints)."""
    c, P, h, src, dst, N = _layer_case()
    E, H = dst.numel(), P["_heads"]
    out0, g0 = _grads_with_hints(c, P, h, src, dst, N, None)
    dis = 0
    for sign in (1.0, -1.0):
        st = {}
        out1, g1 = _grads_with_hints(c, P, h, src, dst, N, {"score": sign * torch.ones(E, H)}, st)
        assert torch.equal(out1, out0)
        for k in g0:
            assert torch.equal(g1[k], g0[k]), k
        assert st["score_near"] == 0
        dis += st["score_disagree"]
    assert dis == E * H


def test_tgat_layer_branch_hint_at_the_score_kink():
    """Scores exactly at the kink (a zero query: z = 0 for every edge) are all in the band,
    and the hint picks the derivative: the query-weight gradient flows through LeakyReLU's
    derivative only, so the positive branch's gradient is exactly 1/slope times the negative
    branch's."""
    c, P, h, src, dst, N = _layer_case()
    E, H = dst.numel(), P["_heads"]
    with torch.no_grad():
        P["w_q.weight"].zero_()
        P["w_q.bias"].zero_()
    st_pos, st_neg = {}, {}
    out_p, gp = _grads_with_hints(c, P, h, src, dst, N, {"score": torch.ones(E, H)}, st_pos)
    out_n, gn = _grads_with_hints(c, P, h, src, dst, N, {"score": -torch.ones(E, H)}, st_neg)
    for st in (st_pos, st_neg):   # a zero query: every term of every score is 0
        assert st["score_zero"] == E * H and st["score_disagree"] == 0
    assert torch.equal(out_p, out_n)   # the value is continuous at the kink
    assert gp["w_q.weight"].abs().max() > 0
    assert torch.allclose(gp["w_q.weight"] * 0.2, gn["w_q.weight"], rtol=1e-12, atol=1e-15)


def test_tgat_layer_branch_hint_at_the_relu_kink():
    """A zero output projection puts every ReLU input at the kink: the output is the
    LayerNorm shift either way; with the ReLU hinted off no gradient reaches w_out, hinted
    on it does, and the deviation statistic measures the hint against the float64 value."""
    c, P, h, src, dst, N = _layer_case()
    D = P["_dims"][3]
    with torch.no_grad():
        P["w_out.weight"].zero_()
        P["w_out.bias"].zero_()
    st_on, st_off = {}, {}
    out_on, g_on = _grads_with_hints(c, P, h, src, dst, N, {"relu": 1e-3 * torch.ones(N, D)}, st_on)
    out_off, g_off = _grads_with_hints(c, P, h, src, dst, N, {"relu": torch.zeros(N, D)}, st_off)
    for st in (st_on, st_off):
        assert st["relu_zero"] == N * D and st["relu_near"] == 0 and st["relu_disagree"] == 0
    beta = P["layer_norm.bias"].detach()
    assert torch.allclose(out_on, beta.expand(N, D)) and torch.allclose(out_off, beta.expand(N, D))
    assert torch.count_nonzero(g_off["w_out.weight"]) == 0
    assert torch.count_nonzero(g_on["w_out.weight"]) > 0
    # |hint - z| / |terms| with z = 0 and terms = 0 everywhere: excluded, so no deviation
    assert st_on["relu_dev"] == 0.0


def test_tgat_layer_zero_edges():
    """layers.py:101-102: a block without edges returns zeros [N, D] (no w_out, no norm)."""
    c, P, h, src, dst, N = _layer_case()
    e = torch.zeros(0, dtype=torch.int64)
    out = ref_cpu.tgat_layer(P, h[:N], torch.zeros(0, 3), torch.zeros(0), e, e, N)
    assert torch.equal(out, torch.zeros(N, P["_dims"][3], dtype=torch.float64))


# ---------------------------------------------------------------------------------------
# counter-based attention dropout (the fused kernels' mask)
# ---------------------------------------------------------------------------------------
def test_dropout_mask_properties():
    n, H = 100_000, 2
    for p in (0.1, 0.5):
        m = C.dropout_mask(n, H, 1234, p)
        scale = np.float32(1.0 / (1.0 - p))
        assert set(np.unique(m).tolist()) <= {0.0, float(scale)}
        keep = (m > 0).mean()
        sd = math.sqrt(p * (1 - p) / m.size)
        assert abs(keep - (1 - p)) < 5 * sd, (p, keep)
        # counter-based: a prefix of a longer mask is the shorter mask
        np.testing.assert_array_equal(C.dropout_mask(1000, H, 1234, p).ravel(), m.ravel()[:2000])
    assert np.all(C.dropout_mask(1000, 2, 7, 0.0) == 1.0)
    a, b = C.dropout_mask(4000, 2, 1, 0.5), C.dropout_mask(4000, 2, 2, 0.5)
    assert 0.4 < (a != b).mean() < 0.6  # independent seeds disagree on about half the entries
    # the high seed word matters as well
    c = C.dropout_mask(4000, 2, 1 + (1 << 32), 0.5)
    assert 0.4 < (a != c).mean() < 0.6


# ---------------------------------------------------------------------------------------
# TGN node memory (memorys.py)
# ---------------------------------------------------------------------------------------
def _state_from(d):
    return {"node_memory": np.asarray(d["node_memory"], dtype=np.float32),
            "node_memory_ts": np.asarray(d["node_memory_ts"], dtype=np.float32),
            "mailbox": np.asarray(d["mailbox"], dtype=np.float32),
            "mailbox_ts": np.asarray(d["mailbox_ts"], dtype=np.float32),
            "next_mail_pos": np.asarray(d["next_mail_pos"], dtype=np.int64)}


def _assert_state_equal(got, want):
    for k in ("node_memory", "node_memory_ts", "mailbox", "mailbox_ts", "next_mail_pos"):
        np.testing.assert_array_equal(got[k], np.asarray(want[k], dtype=got[k].dtype), err_msg=k)


def test_memory_golden():
    """mail_inputs, update_mailbox and update_memory against the row-by-row simulation of
    memorys.py:67-71, 113-139, 86-103 (two batches, repeated roots, 3 slots / 1 slot, with
    and without edge features): every value exact."""
    for c in _load("memory.json")["cases"]:
        N, m, de, slots = c["dims"]
        st = _state_from(c["init"])
        p = c["prep"]
        got = ref_cpu.mail_inputs(st, p["ids"])
        for k in ("mem", "mem_ts", "mem_input", "mail_ts"):
            np.testing.assert_array_equal(got[k], np.asarray(p[k], dtype=np.float32), err_msg=k)
        for b in c["batches"]:
            ef = np.asarray(b["edge_feats"], dtype=np.float32).reshape(len(b["edge_feats"]), de)
            ref_cpu.update_mailbox(st, b["memory"], b["roots"], b["ts"], ef if de else None, b["neg"])
            ref_cpu.update_memory(st, b["nid"], b["memory"], b["lu_ts"], len(b["roots"]), b["neg"])
            _assert_state_equal(st, b["after"])


def test_mail_inputs_invalid_ids_give_zero_rows():
    st = ref_cpu.mailbox_state(5, 2, 1, 2, seed=3)
    got = ref_cpu.mail_inputs(st, [4, -1, 5, 0])
    assert not got["mem"][1].any() and not got["mem"][2].any()
    np.testing.assert_array_equal(got["mem_input"][0], st["mailbox"][4].reshape(-1))
    np.testing.assert_array_equal(got["mail_ts"][3], st["mailbox_ts"][0])


def test_update_mailbox_cycles_the_slots():
    """A node that receives a mail in three consecutive batches fills slots p, p+1, p+2
    (mod slots), each with that batch's mail."""
    st = ref_cpu.mailbox_state(4, 1, 0, 3, seed=1)
    st["next_mail_pos"][:] = 2
    for step in range(3):
        mem = np.array([[10.0 + step], [20.0 + step], [0.0]], dtype=np.float32)
        ref_cpu.update_mailbox(st, mem, [1, 2, 3], [5.0 + step, 6.0 + step, 0.0], None, 1)
    np.testing.assert_array_equal(st["mailbox"][1, :, 0], [11.0, 12.0, 10.0])
    np.testing.assert_array_equal(st["mailbox"][2, :, 0], [21.0, 22.0, 20.0])
    np.testing.assert_array_equal(st["mailbox"][1, :, 1], [21.0, 22.0, 20.0])
    # row r of the interleaved mails takes ts[r]: node 1 (row 0) ts[0], node 2 (row 1) ts[1]
    np.testing.assert_array_equal(st["mailbox_ts"][1], [6.0, 7.0, 5.0])
    np.testing.assert_array_equal(st["mailbox_ts"][2], [7.0, 8.0, 6.0])
    assert st["next_mail_pos"][1] == 2 and st["next_mail_pos"][0] == 2


def _recurrent_params(c, gru):
    P = c["P"]
    t = lambda v: torch.tensor(v, dtype=torch.float64)
    k = ("w_ih", "w_hh", "b_ih", "b_hh") if gru else ("r_ih", "r_hh", "rb_ih", "rb_hh")
    return {"updater.weight_ih": t(P[k[0]]), "updater.weight_hh": t(P[k[1]]),
            "updater.bias_ih": t(P[k[2]]), "updater.bias_hh": t(P[k[3]]),
            "time_enc.w.weight": torch.tensor(P["tw"], dtype=torch.float32).view(-1, 1),
            "time_enc.w.bias": torch.tensor(P["tb"], dtype=torch.float32)}


@pytest.mark.parametrize("gru", [True, False])
def test_recurrent_update_golden(gru):
    c = _load("recurrent.json")
    out = ref_cpu.recurrent_update(_recurrent_params(c, gru), c["mails"], c["h"],
                                   torch.tensor(c["ts"]), torch.tensor(c["mem_ts"]), gru)
    np.testing.assert_allclose(out.numpy(), np.asarray(c["gru" if gru else "rnn"]), rtol=1e-12,
                               atol=1e-13)


@pytest.mark.parametrize("gru", [True, False])
def test_recurrent_update_matches_torch_cells(gru):
    """The written-out cell equals torch.nn.GRUCell / RNNCell (float64) applied to
    [mails, time features]."""
    torch.manual_seed(5)
    n, mail, dt, hid = 7, 10, 6, 5
    cell = (torch.nn.GRUCell if gru else torch.nn.RNNCell)(mail + dt, hid).double()
    P = {"updater." + k: v.detach() for k, v in cell.named_parameters()}
    P["time_enc.w.weight"] = ref_cpu.time_encoding_weight(dt).view(-1, 1)
    P["time_enc.w.bias"] = torch.randn(dt)
    mails, h = torch.randn(n, mail, dtype=torch.float64), torch.randn(n, hid, dtype=torch.float64)
    ts, mem_ts = torch.rand(n) * 1e5, torch.rand(n) * 1e4
    tf = ref_cpu.time_encode(ts - mem_ts, P["time_enc.w.weight"].view(-1), P["time_enc.w.bias"])
    want = cell(torch.cat([mails, tf], 1), h)
    got = ref_cpu.recurrent_update(P, mails, h, ts, mem_ts, gru)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
