"""Host-side logic of fast_amd on the CPU (no kernel launches): the binding's error
behaviour, the operator-flag manager, the block layout, the K-space algebra the fused
kernels rely on, module construction order, the workload generators and bench.py's
single-GPU guard."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import fast_amd
from fast_amd import efficientGOP, tgat, workloads

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
fa = fast_amd.fastAgg


def test_binding_is_the_top_level_fastAgg():
    import fastAgg

    assert fastAgg is fa
    for name in ("forward_edge_softmax", "backward_edge_softmax", "forward_csr_edge_softmax",
                 "backward_csr_edge_softmax", "forward_balanced_edge_softmax",
                 "backward_balanced_edge_softmax", "forward_tgat", "backward_tgat",
                 "forward_tgat_shd", "backward_tgat_shd", "forward_fused_attn",
                 "backward_fused_attn", "exclusive_sum", "cal_deg", "getBalancedPtr"):
        assert callable(getattr(fa, name)), name


@pytest.mark.parametrize("call", [
    lambda: fa.forward_edge_softmax(torch.zeros(3, dtype=torch.int32),
                                    torch.zeros(3, dtype=torch.int32), torch.zeros(4, 2), 512, 2),
    lambda: fa.exclusive_sum(torch.zeros(5, dtype=torch.int32)),
    lambda: fa.cal_deg(torch.zeros(5, dtype=torch.int32), 3),
    lambda: fa.forward_tgat(torch.zeros(4, dtype=torch.int64), torch.zeros(4, dtype=torch.int64),
                            torch.zeros(8, 3), 4, 8, 128),
])
def test_cpu_tensors_are_rejected(call):
    """Same contract as the reference binding (TORCH_CHECK is_cuda, operators.cpp:3-5)."""
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        call()


def test_init_gop_launch_constants():
    """efficientGOP.py:6-38: per-method launch parameters (accepted, not used by gfx950)."""
    fm = efficientGOP.forwardManager()
    fm.init_gop(fast_agg=1, fast_esm=1)
    assert (fm.fastAggFlag, fm.fastESMFlag, fm.aggNodePB, fm.aggFeat) == (1, 1, 8, 128)
    assert (fm.node_num_per_block, fm.reduceSize) == (512, 16)
    fm.init_gop(fast_agg=2, fast_esm=2, csr_out=1)
    assert (fm.aggNodePB, fm.aggFeat, fm.reduceSize, fm.node_num_per_block, fm.CSR_OUT) == (
        8, 32, 16, 32, 1)


def test_block_layout():
    degs = torch.tensor([2, 0, 3, 1])
    b = tgat.Block.from_fanout(4, degs)
    src, dst = b.edges()
    assert b.num_dst_nodes() == 4 and b.num_edges() == 6 and b.num_src_nodes() == 10
    assert src.tolist() == [4, 5, 6, 7, 8, 9]          # edge e comes from source node N + e
    assert dst.tolist() == [0, 0, 2, 2, 2, 3]          # grouped by ascending destination
    assert b.indptr.tolist() == [0, 2, 5, 6]           # CSR over the non-empty destinations
    assert b.indptr.dtype == torch.int32


def test_kspace_absorbs_the_projection():
    """W [x_n | x_e | x_t] + b == to_kspace(W, b) . x_aug, where x_aug pads every part to a
    multiple of 4 and appends the constant 1 of the bias (then 3 zeros)."""
    g = torch.Generator().manual_seed(0)
    for dn, de, dt in ((7, 5, 3), (100, 172, 100), (0, 12, 9), (13, 6, 0), (8, 0, 4)):
        D, E = 6, 11
        W = torch.randn(D, dn + de + dt, generator=g, dtype=torch.float64)
        b = torch.randn(D, generator=g, dtype=torch.float64)
        x = torch.randn(E, dn + de + dt, generator=g, dtype=torch.float64)
        Wk = tgat.to_kspace(W, b, dn, de, dt)
        assert Wk.shape == (D, tgat.kspace_width(dn, de, dt))
        parts, off = [], 0
        for d in (dn, de, dt):
            parts.append(torch.nn.functional.pad(x[:, off:off + d], (0, (-d) % 4)))
            off += d
        one = torch.zeros(E, 4, dtype=torch.float64)
        one[:, 0] = 1.0
        x_aug = torch.cat(parts + [one], 1)
        torch.testing.assert_close(x_aug @ Wk.T, x @ W.T + b, rtol=1e-12, atol=1e-12)


def test_kspace_gradients():
    """to_kspace is a scatter of the weight columns and the bias: its gradient is the
    matching gather (float64 finite differences)."""
    g = torch.Generator().manual_seed(3)
    for dn, de, dt in ((7, 5, 3), (0, 12, 9), (13, 6, 0)):
        W = torch.randn(4, dn + de + dt, generator=g, dtype=torch.float64, requires_grad=True)
        b = torch.randn(4, generator=g, dtype=torch.float64, requires_grad=True)
        assert torch.autograd.gradcheck(lambda w, bb: tgat.to_kspace(w, bb, dn, de, dt), (W, b))


def test_absorbed_attention_equals_per_edge_attention():
    """The fused kernels score q_h . (W_k x + b_k)_h as (Q_h W_k,h) . x_aug and aggregate
    V through xbar = sum_e a_e x_aug,e, out_h = W_v,h xbar_h; with a softmax over one
    destination both orders give the same result (float64, on the CPU)."""
    g = torch.Generator().manual_seed(1)
    dn, de, dt, H, dh, E = 5, 6, 3, 2, 4, 9
    D = H * dh
    Wk, Wv = (torch.randn(D, dn + de + dt, generator=g, dtype=torch.float64) for _ in range(2))
    bk, bv = (torch.randn(D, generator=g, dtype=torch.float64) for _ in range(2))
    x = torch.randn(E, dn + de + dt, generator=g, dtype=torch.float64)
    q = torch.randn(H, dh, generator=g, dtype=torch.float64)
    K = (x @ Wk.T + bk).view(E, H, dh)
    V = (x @ Wv.T + bv).view(E, H, dh)
    s = torch.nn.functional.leaky_relu((K * q[None]).sum(-1), 0.2)
    a = torch.softmax(s, 0)
    out_ref = (a[:, :, None] * V).sum(0)
    # absorbed form
    wk = tgat.to_kspace(Wk, bk, dn, de, dt).view(H, dh, -1)
    wv = tgat.to_kspace(Wv, bv, dn, de, dt).view(H, dh, -1)
    parts, off = [], 0
    for d in (dn, de, dt):
        parts.append(torch.nn.functional.pad(x[:, off:off + d], (0, (-d) % 4)))
        off += d
    bias = torch.zeros(E, 4, dtype=torch.float64)
    bias[:, 0] = 1
    x_aug = torch.cat(parts + [bias], 1)
    qt = torch.einsum("hd,hdk->hk", q, wk)
    s2 = torch.nn.functional.leaky_relu(x_aug @ qt.T, 0.2)
    a2 = torch.softmax(s2, 0)
    xbar = a2.T @ x_aug                      # [H, Kp]
    out = torch.einsum("hdk,hk->hd", wv, xbar)
    torch.testing.assert_close(out, out_ref, rtol=1e-12, atol=1e-12)


def test_fused_kernel_bytes_accounting():
    n, e, dn, de, dt, H = 120_000, 1_200_000, 100, 172, 100, 2
    kp = tgat.kspace_width(dn, de, dt)
    b = tgat.fused_kernel_bytes(n, e, dn, de, dt, H, True, True)
    per_edge = 8 + 8 + 4 + 4 * (dn + de) + 4 * H
    assert b["fwd"] == 4 * (n + 1) + 8 * dt + e * per_edge + n * (8 * H * kp + 8 * H)
    # backward: xbar and dxbar read, dqt written, and of qt the time chunks (25 here) read;
    # with the node-row gradient also qt's node chunks (25) and the rows written
    q_time, q_node = 16 * H * 25, 16 * H * 25
    assert b["bwd"] == 4 * (n + 1) + 8 * dt + e * per_edge + n * (12 * H * kp + q_time + 8 * H)
    assert tgat.fused_kernel_bytes(n, e, dn, de, dt, H, True, True, d_node=True)["bwd"] == \
        b["bwd"] + e * 4 * dn + n * q_node
    # with T = dxbar . xbar given, xbar's rows are replaced by one float per head
    assert tgat.fused_kernel_bytes(n, e, dn, de, dt, H, True, True, tdot=True)["bwd"] == \
        b["bwd"] - n * (4 * H * kp - 4 * H)


def test_layer_construction_order_matches_reference():
    """Same modules, shapes and creation order as layers.py:53-97 (non-combined, fastKQV
    off), so a given torch seed gives the same initial parameters."""
    dn, de, dt, H, D = 100, 172, 100, 2, 100
    torch.manual_seed(42)
    layer = tgat.TransfomerAttentionLayer(dn, de, dt, H, 0.1, 0.1, D)
    torch.manual_seed(42)
    te = torch.nn.Linear(1, dt)
    te.weight = torch.nn.Parameter(torch.from_numpy(
        1 / 10 ** np.linspace(0, 9, dt, dtype=np.float32)).reshape(dt, -1))
    te.bias = torch.nn.Parameter(torch.zeros(dt))
    ref = [("time_enc.w.weight", te.weight), ("time_enc.w.bias", te.bias)]
    for name, fin in (("w_q", dn + dt), ("w_k", dn + de + dt), ("w_v", dn + de + dt),
                      ("w_out", dn + D)):
        lin = torch.nn.Linear(fin, D)
        ref += [(name + ".weight", lin.weight), (name + ".bias", lin.bias)]
    ln = torch.nn.LayerNorm(D)
    ref += [("layer_norm.weight", ln.weight), ("layer_norm.bias", ln.bias)]
    got = list(layer.named_parameters())
    assert [n for n, _ in got] == [n for n, _ in ref]
    for (n, p), (_, r) in zip(got, ref):
        assert torch.equal(p.detach(), r.detach()), n
    assert layer.negative_slope == 0.2


def test_time_encode_module():
    te = tgat.TimeEncode(5)
    t = torch.tensor([0.0, 1.0, 250.0])
    y = te(t)
    assert torch.equal(y[0], torch.ones(5))
    ref = torch.cos(t[:, None].double() * te.w.weight.detach().view(1, -1).double())
    torch.testing.assert_close(y.double(), ref, rtol=0, atol=1e-6)


def test_workloads_are_seeded():
    a = workloads.single_layer(50, seed=3)
    b = workloads.single_layer(50, seed=3)
    assert torch.equal(a.block.edata["dt"], b.block.edata["dt"])
    assert torch.equal(a.block.srcdata["h"], b.block.srcdata["h"])
    c = workloads.single_layer(50, seed=4)
    assert not torch.equal(a.block.edata["dt"], c.block.edata["dt"])
    assert a.block.num_edges() == 500 and bool((a.block.edata["dt"] >= 0).all())


def test_ragged_degrees():
    d = workloads.ragged_degrees(20_000, seed=0)
    assert d.min() >= 0 and d.max() <= 20
    zero = float((d == 0).mean())
    assert 0.03 < zero < 0.08  # about 5 % of the destinations carry no edges


def test_bench_traffic_only_for_unchanged_kernel_sources(tmp_path, monkeypatch):
    """bench.py reports roofline.traffic from a committed rocprofv3 summary only while the
    kernel sources it was measured on are unchanged (the summary records their hash)."""
    import shutil

    import bench

    for rel in bench.TRAFFIC_SOURCES:
        (tmp_path / rel).parent.mkdir(parents=True, exist_ok=True)
        shutil.copy(os.path.join(ROOT, rel), tmp_path / rel)
    (tmp_path / "profiles").mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    prof = tmp_path / "profiles" / "tgat_C9_pmc_traffic.md"
    assert bench.measured_traffic("c9", "tgat_bwd")[0] is None          # no summary
    prof.write_text(f"source_sha {bench.source_hash()}\ntraffic_per_launch tgat_bwd 123\n")
    assert bench.measured_traffic("c9", "tgat_bwd")[0] == 123
    assert bench.measured_traffic("c9", "tgat_fwd")[0] is None          # kernel not listed
    src = tmp_path / bench.TRAFFIC_SOURCES[0]
    src.write_text(src.read_text() + "\n// edited\n")
    value, note = bench.measured_traffic("c9", "tgat_bwd")
    assert value is None and "other kernel sources" in note


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)


class _FakeSample:
    """A sampler result with the FAST sampler's accessors (sampler_core.cpp): dim_out
    destinations, `deg` edges each, edge e from source node dim_out + e."""

    def __init__(self, dim_out, deg, seed):
        rng = np.random.default_rng(seed)
        E = dim_out * deg
        self._row = np.repeat(np.arange(dim_out, dtype=np.int32), deg)
        self._col = np.arange(dim_out, dim_out + E, dtype=np.int32)
        self._nodes = rng.integers(0, 10 ** 6, dim_out + E).astype(np.int64)
        self._ts = rng.random(dim_out + E).astype(np.float32)
        self._dts = rng.random(dim_out + E).astype(np.float32)
        self._eid = rng.integers(0, 10 ** 7, E).astype(np.int64)
        self._n = (dim_out + E, dim_out)

    def row(self): return self._row
    def col(self): return self._col
    def nodes(self): return self._nodes
    def ts(self): return self._ts
    def dts(self): return self._dts
    def eid(self): return self._eid
    def dim_in(self): return self._n[0]
    def dim_out(self): return self._n[1]


def test_to_blocks_mirrors_to_dgl_blocks():
    """utils.py:67-87: edges col -> row, dt = dts[num_dst:], ids and ts on the sources, the
    results grouped `hist` at a time and the groups reversed; reverse=True swaps the roles."""
    from fast_amd.mfg import to_blocks

    ret = [_FakeSample(5, 3, 0), _FakeSample(2, 4, 1), _FakeSample(3, 2, 2), _FakeSample(4, 1, 3)]
    groups = to_blocks(ret, hist=2, device="cpu")
    assert [len(g) for g in groups] == [2, 2]
    assert groups[0][0].num_dst_nodes() == 3 and groups[1][0].num_dst_nodes() == 5
    b, r = groups[1][0], ret[0]
    src, dst = b.edges()
    assert torch.equal(src, torch.from_numpy(r.col()).long())
    assert torch.equal(dst, torch.from_numpy(r.row()).long())
    assert b.num_src_nodes() == r.dim_in() and b.num_edges() == 15
    assert torch.equal(b.srcdata["ID"], torch.from_numpy(r.nodes()))
    assert torch.equal(b.srcdata["ts"], torch.from_numpy(r.ts()))
    assert torch.equal(b.edata["dt"], torch.from_numpy(r.dts())[5:])
    assert torch.equal(b.edata["ID"], torch.from_numpy(r.eid()))
    rb = to_blocks(ret[:1], device="cpu", reverse=True)[0][0]
    s2, d2 = rb.edges()
    assert torch.equal(s2, torch.from_numpy(r.row()).long()) and rb.num_dst_nodes() == r.dim_in()
    assert torch.equal(rb.dstdata["ID"], torch.from_numpy(r.nodes()))
    assert torch.equal(rb.edata["dt"], torch.from_numpy(r.dts())[r.dim_out():])


def test_to_blocks_on_host_match_restatement():
    """fast_amd.mfg.to_blocks on the host equals the oracle's restatement of utils.py:67-87
    on the golden fixture's sampler results (ragged degrees, zero-degree destinations), for
    both directions and hist 1 and 2."""
    from fast_amd.mfg import to_blocks
    from oracle.ref_cpu import to_dgl_blocks
    from tests.test_oracle import _GoldenSample, _load

    ret = [_GoldenSample(d) for d in _load("mfg.json")["results"]]
    for hist in (1, 2):
        for rev in (False, True):
            got = to_blocks(ret, hist=hist, reverse=rev, device="cpu")
            want = to_dgl_blocks(ret, hist, reverse=rev)
            assert [len(g) for g in got] == [len(g) for g in want]
            for gg, gw in zip(got, want):
                for b, w in zip(gg, gw):
                    _assert_block_matches(b, w)


def _assert_block_matches(b, w):
    src, dst = b.edges()
    np.testing.assert_array_equal(src.cpu().numpy(), w["src"])
    np.testing.assert_array_equal(dst.cpu().numpy(), w["dst"])
    assert (b.num_src_nodes(), b.num_dst_nodes()) == (w["num_src"], w["num_dst"])
    side = b.srcdata if w["node_side"] == "src" else b.dstdata
    np.testing.assert_array_equal(side["ID"].cpu().numpy(), w["ID"])
    np.testing.assert_array_equal(side["ts"].cpu().numpy(), w["ts"])
    np.testing.assert_array_equal(b.edata["dt"].cpu().numpy(), w["dt"])
    np.testing.assert_array_equal(b.edata["ID"].cpu().numpy(), w["eID"])


def test_split_rows_backward_fills_the_rows_in_front():
    """_SplitRows.backward: when the edge-row gradient is rows n.. of a full-size tensor (the
    fused backward's d_node_front), the destination-row gradient goes into the rows in front
    and that tensor is the result (no concatenation); any other gradient is concatenated."""
    class Ctx:
        n, shape = 4, (10, 3)

    gen = torch.Generator().manual_seed(0)
    full = torch.zeros(10, 3)
    g_src = full[4:]
    g_src.copy_(torch.randn(6, 3, generator=gen))
    g_dst = torch.randn(4, 3, generator=gen)
    want = torch.cat([g_dst, g_src])
    out, _ = tgat._SplitRows.backward(Ctx(), g_dst, g_src)
    assert out.data_ptr() == full.data_ptr() and torch.equal(out, want)
    out2, _ = tgat._SplitRows.backward(Ctx(), g_dst, g_src.clone())
    assert torch.equal(out2, want)
    out3, _ = tgat._SplitRows.backward(Ctx(), None, g_src.clone())
    assert torch.equal(out3[:4], torch.zeros(4, 3)) and torch.equal(out3[4:], g_src)


# ---------------------------------------------------------------------------------------
# TGN node memory: host-side state and dispatch (no kernels)
# ---------------------------------------------------------------------------------------
def _mem_param(**kw):
    p = {"type": "node", "dim_time": 100, "deliver_to": "self", "mail_combine": "last",
         "memory_update": "gru", "mailbox_size": 2, "combine_node_feature": True, "dim_out": 100}
    p.update(kw)
    return p


def test_mailbox_state_matches_the_reference_layout():
    """memorys.py:13-18: the tensors, shapes and dtypes a MailBox holds, zero-initialised on
    the host until moved."""
    from fast_amd.memorys import MailBox

    mb = MailBox(_mem_param(), 11, 172)
    assert mb.node_memory.shape == (11, 100) and mb.node_memory.dtype == torch.float32
    assert mb.node_memory_ts.shape == (11,)
    assert mb.mailbox.shape == (11, 2, 372) and mb.mailbox_ts.shape == (11, 2)
    assert mb.next_mail_pos.dtype == torch.long and mb.device.type == "cpu"
    for t in (mb.node_memory, mb.mailbox, mb.mailbox_ts, mb.next_mail_pos):
        assert not t.any()
    with pytest.raises(NotImplementedError):
        MailBox(_mem_param(type="none"), 3, 0)


def test_mailbox_unsupported_modes_raise():
    from fast_amd.memorys import MailBox

    mb = MailBox(_mem_param(deliver_to="neighbors"), 4, 0)
    with pytest.raises(NotImplementedError):
        mb.update_mailbox(None, torch.zeros(3, 100), np.zeros(3, np.int32), np.zeros(3, np.float32),
                          None, None)
    mb = MailBox(_mem_param(mail_combine="mean"), 4, 0)
    with pytest.raises(NotImplementedError):
        mb.update_mailbox(None, torch.zeros(3, 100), np.zeros(3, np.int32), np.zeros(3, np.float32),
                          None, None)


def test_mailbox_write_tags_wrap_before_32_bits():
    """The per-node tags of the write-back grow by one generation per call and restart
    (with the tags cleared) before the generation would pass 32 bits."""
    from fast_amd import memorys

    mb = memorys.MailBox(_mem_param(), 5, 0)
    last, g1 = mb._tags()
    _, g2 = mb._tags()
    assert (g1, g2) == (1, 2) and last.shape == (5,) and last.dtype == torch.int64
    mb._gen = memorys._TAG_LIMIT - 1
    last.fill_(7)
    last2, g = mb._tags()
    assert g == 1 and not last2.any()


def test_updaters_keep_the_reference_parameters():
    """GRUMemeoryUpdater / RNNMemeoryUpdater hold the reference's modules (state-dict keys
    and shapes of memorys.py:270-282, 308-320)."""
    from fast_amd.memorys import GRUMemeoryUpdater, RNNMemeoryUpdater

    g = GRUMemeoryUpdater(_mem_param(), 372, 100, 100, 50)
    sd = {k: tuple(v.shape) for k, v in g.state_dict().items()}
    assert sd["updater.weight_ih"] == (300, 472) and sd["updater.weight_hh"] == (300, 100)
    assert sd["time_enc.w.weight"] == (100, 1) and sd["node_feat_map.weight"] == (100, 50)
    r = RNNMemeoryUpdater(_mem_param(), 372, 100, 0, 100)
    sd = {k: tuple(v.shape) for k, v in r.state_dict().items()}
    assert sd == {"updater.weight_ih": (100, 372), "updater.weight_hh": (100, 100),
                  "updater.bias_ih": (100,), "updater.bias_hh": (100,)}
