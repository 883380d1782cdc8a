"""TGN node memory on the GPU (fast_amd.memorys over the memory kernels) against the CPU
restatement (oracle/ref_cpu.py, memorys.py:6-304).

Gathers and write-backs are copies: bit-exact. The updater is float32 on the GPU against
the float64 restatement: outputs and every parameter gradient within 1e-5 (relative, whole
tensor). Sizes are small enough for the oracle to finish in seconds.
"""
import numpy as np
import pytest
import torch

from oracle import ref_cpu
from tests._util import FP32_TOL, assert_equal, assert_rel

pytestmark = pytest.mark.gpu


def _param(m, de, slots, dt=100):
    return {"type": "node", "dim_time": dt, "deliver_to": "self", "mail_combine": "last",
            "memory_update": "gru", "mailbox_size": slots, "combine_node_feature": True,
            "dim_out": m}


def _mailbox(dev, st, param, de):
    from fast_amd.memorys import MailBox

    t = lambda a: torch.from_numpy(a.copy()).to(dev)
    return MailBox(param, st["node_memory"].shape[0], de, _node_memory=t(st["node_memory"]),
                   _node_memory_ts=t(st["node_memory_ts"]), _mailbox=t(st["mailbox"]),
                   _mailbox_ts=t(st["mailbox_ts"]), _next_mail_pos=t(st["next_mail_pos"]))


def _assert_state(mb, st):
    for k, got in (("node_memory", mb.node_memory), ("node_memory_ts", mb.node_memory_ts),
                   ("mailbox", mb.mailbox), ("mailbox_ts", mb.mailbox_ts),
                   ("next_mail_pos", mb.next_mail_pos)):
        assert_equal(got.reshape(-1), torch.from_numpy(st[k]).reshape(-1), k)


class _B:
    """The block fields the memory path reads and writes."""

    def __init__(self, ids, ts, h=None):
        self.srcdata = {"ID": ids, "ts": ts}
        if h is not None:
            self.srcdata["h"] = h


@pytest.mark.parametrize("m,de,slots", [(100, 172, 1), (3, 2, 3), (8, 0, 2)])
@pytest.mark.parametrize("id_dtype", [torch.int32, torch.int64])
def test_prep_input_mails_matches_oracle(dev, m, de, slots, id_dtype):
    """Every gathered row, time and mail bit-exact (16-byte and scalar copy paths); ids
    repeat."""
    N = 700
    st = ref_cpu.mailbox_state(N, m, de, slots, seed=m + slots)
    mb = _mailbox(dev, st, _param(m, de, slots), de)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, N, 2500)
    ids[:50] = ids[50:100]
    b = _B(torch.from_numpy(ids).to(id_dtype).to(dev), torch.zeros(len(ids), device=dev))
    mb.prep_input_mails([b])
    want = ref_cpu.mail_inputs(st, ids)
    for k in ("mem", "mem_ts", "mem_input", "mail_ts"):
        assert_equal(b.srcdata[k].reshape(-1), torch.from_numpy(want[k]).reshape(-1), k)
    rows = b.srcdata["_mem_rows"]
    assert rows.shape == (len(ids), slots * (2 * m + de) + 100)


def test_mail_gather_ids_outside_the_table_give_zero_rows(dev):
    from fast_amd import fastAgg

    st = ref_cpu.mailbox_state(50, 4, 4, 2, seed=9)
    t = lambda a: torch.from_numpy(a).to(dev)
    ids = np.array([3, -1, 50, 49, 10**6, 0], dtype=np.int64)
    mem, mem_ts, x, mail_ts = fastAgg.mail_gather(t(ids), t(st["node_memory"]), t(st["node_memory_ts"]),
                                                  t(st["mailbox"]), t(st["mailbox_ts"]), 24)
    want = ref_cpu.mail_inputs(st, ids)
    assert_equal(mem.reshape(-1), torch.from_numpy(want["mem"]).reshape(-1), "mem")
    assert_equal(x[:, :24].reshape(-1), torch.from_numpy(want["mem_input"]).reshape(-1), "mails")
    assert_equal(mail_ts.reshape(-1), torch.from_numpy(want["mail_ts"]).reshape(-1), "mail_ts")


def test_time_rows_and_gradient(dev):
    """cos(w (ts - mem_ts) + b) with the argument rounded as float32 Linear(1, dt), against
    the float64 cosine of that argument (including arguments past 2^22, which take the
    library cosine); dw, db against float64 sums."""
    from fast_amd import fastAgg

    rng = np.random.default_rng(2)
    n, dt = 3000, 100
    ts = (rng.random(n) * 1e6).astype(np.float32)
    mem_ts = (rng.random(n) * 1e5).astype(np.float32)
    ts[:5] = 8e6
    mem_ts[:5] = 0
    w = ref_cpu.time_encoding_weight(dt)
    b = torch.from_numpy(rng.standard_normal(dt).astype(np.float32))
    out = torch.zeros(n, dt + 7, device=dev)
    T, M = torch.from_numpy(ts), torch.from_numpy(mem_ts)
    fastAgg.time_rows_(out, 3, T.to(dev), M.to(dev), w.to(dev), b.to(dev))
    want = ref_cpu.time_encode(T - M, w, b)
    assert float((out[:, 3:3 + dt].cpu().double() - want).abs().max()) < 5e-7
    assert not out[:, :3].any() and not out[:, 3 + dt:].any()
    g = torch.randn(n, dt, dtype=torch.float64)
    w64, b64 = w.double().requires_grad_(True), b.double().requires_grad_(True)
    (ref_cpu.time_encode(T - M, w64, b64) * g).sum().backward()
    dw, db = fastAgg.time_rows_grad(g.float().to(dev), T.to(dev), M.to(dev), w.to(dev), b.to(dev))
    assert_rel(dw, w64.grad, FP32_TOL, "dw")
    assert_rel(db, b64.grad, FP32_TOL, "db")


def _updater(kind, m, de, dt, dim_node):
    from fast_amd.memorys import GRUMemeoryUpdater, RNNMemeoryUpdater

    cls = GRUMemeoryUpdater if kind == "gru" else RNNMemeoryUpdater
    return cls(_param(m, de, 1, dt), 2 * m + de, m, dt, dim_node)


def _oracle_params(mod):
    return {k: v.detach().cpu().double().requires_grad_(True) for k, v in mod.named_parameters()}


@pytest.mark.parametrize("kind", ["gru", "rnn"])
@pytest.mark.parametrize("dt,dim_node", [(100, 0), (100, 100), (100, 50), (0, 0)])
def test_updater_matches_oracle(dev, kind, dt, dim_node):
    """prep_input_mails + updater forward (memorys.py:286-304) and the backward of a loss on
    srcdata['h']: the updated memory, h and the gradient of every parameter (cell, time
    encoder, node-feature map) within 1e-5 of the float64 restatement."""
    torch.manual_seed(3)
    m, de, slots = 100, 172, 1
    N, n = 5000, 4000
    st = ref_cpu.mailbox_state(N, m, de, slots, seed=4)
    mp = _param(m, de, slots, dt)
    mb = _mailbox(dev, st, mp, de)
    upd = _updater(kind, m, de, dt, dim_node).to(dev)
    rng = np.random.default_rng(5)
    ids = rng.integers(0, N, n)
    ts = (st["node_memory_ts"][ids] + rng.exponential(1e4, n)).astype(np.float32)
    h0 = torch.randn(n, dim_node) if dim_node else None
    b = _B(torch.from_numpy(ids).to(dev), torch.from_numpy(ts).to(dev),
           h0.to(dev) if h0 is not None else None)
    mb.prep_input_mails([b])
    upd([b])
    G = torch.randn(n, m)
    (b.srcdata["h"] * G.to(dev)).sum().backward()

    P = _oracle_params(upd)
    got_in = ref_cpu.mail_inputs(st, ids)
    ref = ref_cpu.recurrent_update(P, got_in["mem_input"], got_in["mem"], torch.from_numpy(ts),
                                   torch.from_numpy(got_in["mem_ts"]), kind == "gru")
    h_ref = ref_cpu.combine_node_feature(P, h0, ref, dim_node, m)
    (h_ref * G.double()).sum().backward()
    assert_rel(upd.last_updated_memory, ref, FP32_TOL, "updated memory")
    assert_rel(b.srcdata["h"], h_ref, FP32_TOL, "h")
    assert b.srcdata["mem_input"].shape == (n, slots * (2 * m + de) + dt)
    for name, prm in upd.named_parameters():
        assert_rel(prm.grad, P[name].grad, FP32_TOL, f"grad {name}")
    assert_equal(upd.last_updated_nid, torch.from_numpy(ids).to(dev), "nid")


@pytest.mark.parametrize("de,slots", [(172, 1), (0, 3), (5, 2)])
def test_write_back_matches_oracle(dev, de, slots):
    """Four batches of update_mailbox then update_memory (train.py:220-221) with roots drawn
    from a small id range (repeats within and across batches): the whole state bit-exact."""
    m, N = 100, 3000
    st = ref_cpu.mailbox_state(N, m, de, slots, seed=6)
    mb = _mailbox(dev, st, _param(m, de, slots), de)
    rng = np.random.default_rng(7)
    for step in range(4):
        n, neg = 600, 1
        roots = rng.integers(0, 400, n * (neg + 2)).astype(np.int32)
        ts = (rng.random(len(roots)) * 1e6).astype(np.float32)
        rows = len(roots) + 100
        memory = rng.standard_normal((rows, m)).astype(np.float32)
        nid = np.concatenate([roots, rng.integers(0, N, 100)]).astype(np.int64)
        lu_ts = (rng.random(rows) * 1e6).astype(np.float32)
        ef = rng.standard_normal((n, de)).astype(np.float32) if de else None
        mb.update_mailbox(torch.from_numpy(nid).to(dev), torch.from_numpy(memory).to(dev), roots, ts,
                          torch.from_numpy(ef).to(dev) if de else None, None, neg_samples=neg)
        mb.update_memory(torch.from_numpy(nid).to(dev), torch.from_numpy(memory).to(dev), roots,
                         torch.from_numpy(lu_ts).to(dev), neg_samples=neg)
        ref_cpu.update_mailbox(st, memory, roots, ts, ef, neg)
        ref_cpu.update_memory(st, nid, memory, lu_ts, len(roots), neg)
        _assert_state(mb, st)


def test_write_back_with_host_state_moves_it_to_the_gpu(dev):
    """A MailBox built on the host (the reference's default placement) is moved to the GPU
    on first use and then updated there."""
    from fast_amd.memorys import MailBox

    mb = MailBox(_param(4, 0, 1), 10, 0)
    assert mb.node_memory.device.type == "cpu"
    roots = np.array([1, 2, 3], dtype=np.int32)
    mem = torch.arange(12, dtype=torch.float32).reshape(3, 4).to(dev)
    mb.update_mailbox(None, mem, roots, np.array([5.0, 6.0, 7.0], dtype=np.float32), None, None)
    mb.update_memory(torch.from_numpy(roots).to(dev), mem, roots,
                     torch.tensor([5.0, 6.0, 7.0], device=dev))
    assert mb.node_memory.device.type == "cuda"
    assert_equal(mb.mailbox[1, 0].cpu(), torch.tensor([0, 1, 2, 3, 4, 5, 6, 7], dtype=torch.float32), "mail src")
    assert_equal(mb.mailbox[2, 0].cpu(), torch.tensor([4, 5, 6, 7, 0, 1, 2, 3], dtype=torch.float32), "mail dst")
    assert_equal(mb.node_memory[1:3].cpu().reshape(-1), mem[:2].cpu().reshape(-1), "memory")


def test_tgn_step_matches_oracle(dev):
    """One TGN step on a ragged block: prep_input_mails, the GRU updater writing
    srcdata['h'], the fused TGAT layer on it, the backward of a loss on the layer output, then
    update_mailbox / update_memory. The layer output and every gradient (layer and updater)
    within 1e-5 of the float64 restatement chain; the written state bit-exact."""
    from fast_amd.tgat import Block, TransfomerAttentionLayer

    torch.manual_seed(8)
    m, de, dt, H = 100, 172, 100, 2
    N_nodes = 4000
    st = ref_cpu.mailbox_state(N_nodes, m, de, 1, seed=10)
    mp = _param(m, de, 1, dt)
    mb = _mailbox(dev, st, mp, de)
    upd = _updater("gru", m, de, dt, 0).to(dev)
    layer = TransfomerAttentionLayer(m, de, dt, H, 0.0, 0.0, m).to(dev)
    rng = np.random.default_rng(11)
    degs = np.minimum(rng.zipf(1.5, 600), 20)
    degs[::20] = 0
    n_roots = 600          # 200 sources, 200 destinations, 200 negatives
    blk = Block.from_fanout(n_roots, torch.from_numpy(degs))
    E = blk.num_edges()
    ids = rng.integers(0, N_nodes, n_roots + E)
    ts = (rng.random(n_roots + E) * 1e6).astype(np.float32)
    f = torch.randn(E, de)
    dtv = torch.from_numpy(rng.exponential(1e4, E).astype(np.float32))
    blk.srcdata["ID"] = torch.from_numpy(ids)
    blk.srcdata["ts"] = torch.from_numpy(ts)
    blk.edata["f"] = f
    blk.edata["dt"] = dtv
    g = blk.to(dev)
    mb.prep_input_mails([g])
    upd([g])
    out = layer(g)
    dout = torch.randn(n_roots, m)
    out.backward(dout.to(dev))

    Pu = _oracle_params(upd)
    Pl = ref_cpu.layer_params(layer)
    inp = ref_cpu.mail_inputs(st, ids)
    h_ref = ref_cpu.recurrent_update(Pu, inp["mem_input"], inp["mem"], torch.from_numpy(ts),
                                     torch.from_numpy(inp["mem_ts"]), True)
    src, dst = blk.edges()
    out_ref = ref_cpu.tgat_layer(Pl, h_ref, f, dtv, src, dst, n_roots)
    out_ref.backward(dout.double())
    assert_rel(out, out_ref, FP32_TOL, "layer output")
    for name, prm in upd.named_parameters():
        assert_rel(prm.grad, Pu[name].grad, FP32_TOL, f"updater grad {name}")
    for name, prm in layer.named_parameters():
        assert_rel(prm.grad, Pl[name].grad, FP32_TOL, f"layer grad {name}")

    roots = ids[:n_roots].astype(np.int32)
    ef = torch.randn(n_roots // 3, de)
    mb.update_mailbox(upd.last_updated_nid, upd.last_updated_memory, roots, ts[:n_roots], ef.to(dev), None)
    mb.update_memory(upd.last_updated_nid, upd.last_updated_memory, roots, upd.last_updated_ts)
    mem32 = upd.last_updated_memory.cpu().numpy()
    ref_cpu.update_mailbox(st, mem32, roots, ts[:n_roots], ef.numpy(), 1)
    ref_cpu.update_memory(st, ids, mem32, ts, n_roots, 1)
    _assert_state(mb, st)
