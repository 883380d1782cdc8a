"""TGN node memory on the GPU: the reference's MailBox and memory updaters (memorys.py:6-304)
with the same class names, constructor arguments, methods and block fields, over the gfx950
kernels of libfastagg_hip.so.

* ``MailBox.prep_input_mails`` gathers every source row's memory, mails and times by node id
  in one kernel (``fastAgg.mail_gather``). The mails are written into rows that already hold
  room for the updater's time features, so the updater never concatenates.
* ``GRUMemeoryUpdater`` / ``RNNMemeoryUpdater`` keep ``torch.nn.GRUCell`` / ``RNNCell`` as
  the parameter holders (same state-dict keys). Their forward is one autograd node: the time
  columns (``fastAgg.time_rows_``), the two input products on the split-bf16 reduce kernel
  (``fastAgg.head_reduce``, without their biases), the gate arithmetic with the biases
  (``fastAgg.gru_fwd`` / ``rnn_fwd``); the backward runs the gate gradients, the weight
  gradients (``fastAgg.head_wgrad``) and the time-encoder gradient
  (``fastAgg.time_rows_grad``).
* ``update_memory`` / ``update_mailbox`` (deliver_to 'self', mail_combine 'last') write back
  with one winner per node id, the row that comes last in the reference's order
  (``fastAgg.memory_update_`` / ``mailbox_update_``). For ``update_memory`` the reference's
  device index_put leaves the winner among repeated ids unspecified; here it is always the
  last row.

The state lives in HBM. A MailBox built on the host (the reference's default) is moved to
the GPU on first use; there is no host path for the gathers or the write-back.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import fastAgg
from . import tgat
from .tgat import TimeEncode

_TAG_LIMIT = 1 << 32


def _timed(name, nbytes, fn, *args):
    """fn(*args), timed (with its algorithmic bytes) when the kernel timer is set."""
    return tgat._timed(name, nbytes, fn, *args)


def _tmm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """a^T b for a [n, p], b [n, q] over many rows (the cells' weight gradients): the per-head
    weight-gradient kernel (split-bf16 matrix-core products, fixed-order sums) with a's
    columns in G groups of at most 128 (one j group of the kernel's workgroup each) and
    every group reading the same rows of b."""
    n, p = a.shape
    q = b.shape[1]
    G = next(g for g in range(1, p + 1) if p % g == 0 and p // g <= 128)
    nb = 4 * (n * p + n * q + p * q)
    y = b.unsqueeze(0).expand(G, n, q)
    return _timed("cell_wgrad", nb, fastAgg.head_wgrad, a, y, G, False).reshape(p, q)


def _as_device(x, device, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(x)) if isinstance(x, np.ndarray) else x
    t = t.to(device=device, non_blocking=False)
    if dtype is not None and t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()


def _ids(x, device) -> torch.Tensor:
    t = _as_device(x, device)
    if t.dtype not in (torch.int32, torch.int64):
        t = t.long()
    return t.reshape(-1)


class MailBox:
    """memorys.py:6-268 for node memory (``memory_param['type'] == 'node'``)."""

    def __init__(self, memory_param, num_nodes, dim_edge_feat, _node_memory=None,
                 _node_memory_ts=None, _mailbox=None, _mailbox_ts=None, _next_mail_pos=None,
                 _update_mail_pos=None):
        self.memory_param = memory_param
        self.dim_edge_feat = dim_edge_feat
        if memory_param["type"] != "node":
            raise NotImplementedError
        m, slots = memory_param["dim_out"], memory_param["mailbox_size"]
        z = torch.zeros
        self.node_memory = z((num_nodes, m), dtype=torch.float32) if _node_memory is None else _node_memory
        self.node_memory_ts = z(num_nodes, dtype=torch.float32) if _node_memory_ts is None else _node_memory_ts
        self.mailbox = (z((num_nodes, slots, 2 * m + dim_edge_feat), dtype=torch.float32)
                        if _mailbox is None else _mailbox)
        self.mailbox_ts = z((num_nodes, slots), dtype=torch.float32) if _mailbox_ts is None else _mailbox_ts
        self.next_mail_pos = z(num_nodes, dtype=torch.long) if _next_mail_pos is None else _next_mail_pos
        self.update_mail_pos = _update_mail_pos
        self.device = self.node_memory.device
        self._last: Optional[torch.Tensor] = None   # per-node write tags of the write-back
        self._gen = 0

    # -- state --------------------------------------------------------------------------
    def reset(self):
        self.node_memory.fill_(0)
        self.node_memory_ts.fill_(0)
        self.mailbox.fill_(0)
        self.mailbox_ts.fill_(0)
        self.next_mail_pos.fill_(0)

    def move_to_gpu(self):
        dev = torch.device("cuda:0")
        self.node_memory = self.node_memory.to(dev)
        self.node_memory_ts = self.node_memory_ts.to(dev)
        self.mailbox = self.mailbox.to(dev)
        self.mailbox_ts = self.mailbox_ts.to(dev)
        self.next_mail_pos = self.next_mail_pos.to(dev)
        if self.update_mail_pos is not None:
            self.update_mail_pos = self.update_mail_pos.to(dev)
        self.device = dev
        self._last = None

    def _ensure_gpu(self):
        if self.device.type != "cuda":
            self.move_to_gpu()

    def _tags(self):
        """(per-node tag array, the next generation) for one write-back call."""
        if self._last is None or self._last.device != self.device:
            self._last = torch.zeros(self.node_memory.shape[0], dtype=torch.int64, device=self.device)
            self._gen = 0
        self._gen += 1
        if self._gen >= _TAG_LIMIT:
            self._last.zero_()
            self._gen = 1
        return self._last, self._gen

    def allocate_pinned_memory_buffers(self, sample_param, batch_size):
        """Kept for the reference's API (memorys.py:38-50). The state is in HBM, so the mail
        gather never stages through host buffers and these stay unused."""
        limit = int(batch_size * 3.3)
        if "neighbor" in sample_param:
            for i in sample_param["neighbor"]:
                limit *= i + 1
        self.pinned_limit = limit

    # -- inputs of the memory updater ---------------------------------------------------
    def _time_dim(self) -> int:
        return int(self.memory_param.get("dim_time", 0) or 0)

    def prep_input_mails(self, mfg, CTdata=None, use_pinned_buffers=False):
        """memorys.py:52-71: b.srcdata 'mem', 'mem_ts', 'mem_input' ([n, slots*mail]) and
        'mail_ts' for every block of the hop."""
        self._ensure_gpu()
        mail_w = self.mailbox.shape[1] * self.mailbox.shape[2]
        width = mail_w + self._time_dim()
        for b in mfg:
            ids = _ids(b.srcdata["ID"], self.device)
            n, m, slots = ids.numel(), self.node_memory.shape[1], self.mailbox.shape[1]
            nbytes = n * (ids.element_size() + 2 * 4 * (m + 1 + mail_w + slots))
            mem, mem_ts, rows, mail_ts = _timed(
                "mail_gather", nbytes, fastAgg.mail_gather, ids, self.node_memory,
                self.node_memory_ts, self.mailbox, self.mailbox_ts, width)
            b.srcdata["mem"] = mem
            b.srcdata["mem_ts"] = mem_ts
            b.srcdata["mem_input"] = rows[:, :mail_w]
            b.srcdata["mail_ts"] = mail_ts
            b.srcdata["_mem_rows"] = rows   # the same rows with room for the time features

    def prep_input_mails_sc(self, mfg, NODE_UV=None):
        """memorys.py:73-84: the same fields; NODE_UV (unique ids, inverse) is returned as
        the reference computes it. The rows are gathered by id directly, which gives the
        values the reference's gather-then-expand gives."""
        self._ensure_gpu()
        for b in mfg:
            if NODE_UV is None:
                NODE_UV = [None, None]
                NODE_UV[0], NODE_UV[1] = torch.unique(b.srcdata["ID"], return_inverse=True)
            if NODE_UV[0].device.type == "cuda":
                NODE_UV[0] = NODE_UV[0].cpu()
        self.prep_input_mails(mfg)
        return NODE_UV

    # -- write-back ---------------------------------------------------------------------
    def update_memory(self, nid, memory, root_nodes, ts, neg_samples=1):
        """memorys.py:86-103: node_memory / node_memory_ts of the first 2n rows (the batch's
        true sources and destinations); the last row of a repeated id wins."""
        if nid is None:
            return
        self._ensure_gpu()
        k = len(root_nodes) // (neg_samples + 2) * 2
        with torch.no_grad():
            ids = _ids(nid[:k], self.device)
            mem = _as_device(memory[:k], self.device, torch.float32)
            t = _as_device(ts[:k], self.device, torch.float32)
            last, gen = self._tags()
            m = mem.shape[1]
            # ids, rows and times read, one row and time written per distinct id (<= k)
            nbytes = k * (ids.element_size() + 4 * m + 4 + 8) + k * (4 * m + 4)
            _timed("memory_update", nbytes, fastAgg.memory_update_, ids, mem, t, self.node_memory,
                   self.node_memory_ts, last, gen)

    def update_mailbox(self, nid, memory, root_nodes, ts, edge_feats, block, neg_samples=1):
        """memorys.py:105-182 for deliver_to 'self' with mail_combine 'last' (TGN, JODIE):
        the mails [mem_self, mem_other, edge_feats] of the batch's true edges, interleaved
        source / destination, the last mail of a node kept."""
        if self.memory_param["deliver_to"] != "self":
            raise NotImplementedError("deliver_to 'neighbors' (APAN) is not built here")
        if self.memory_param["mail_combine"] != "last":
            raise NotImplementedError("mail_combine " + str(self.memory_param["mail_combine"]))
        self._ensure_gpu()
        n = len(root_nodes) // (neg_samples + 2)
        with torch.no_grad():
            roots = _ids(root_nodes, self.device)
            mem = _as_device(memory[:2 * n], self.device, torch.float32)
            t = _as_device(ts[:2 * n], self.device, torch.float32)
            ef = None
            if self.dim_edge_feat > 0:
                ef = _as_device(edge_feats[:n], self.device, torch.float32)
            last, gen = self._tags()
            m, de = mem.shape[1], self.dim_edge_feat
            # per write row: its id, two memory rows, the edge row, its time read; one mail,
            # time and position written per distinct node (<= 2n)
            nbytes = 2 * n * (roots.element_size() + 8 * m + 4 * de + 4 + 8) + 2 * n * (4 * (2 * m + de) + 12)
            _timed("mailbox_update", nbytes, fastAgg.mailbox_update_, roots[:n].contiguous(),
                   roots[n:2 * n].contiguous(), mem, ef, t, self.mailbox, self.mailbox_ts,
                   self.next_mail_pos, last, gen)

    def update_next_mail_pos(self):
        """memorys.py:184-188."""
        if self.update_mail_pos is not None:
            nid = torch.where(self.update_mail_pos == 1)[0]
            self.next_mail_pos[nid] = torch.remainder(self.next_mail_pos[nid] + 1,
                                                      self.memory_param["mailbox_size"])
            self.update_mail_pos.fill_(0)

    # -- split write-back (the reference's distributed trainer) ---------------------------
    @staticmethod
    def _last_rows(ids: torch.Tensor) -> torch.Tensor:
        """Row index of the last occurrence of every distinct id, in ascending id order."""
        uni, inv = torch.unique(ids, return_inverse=True)
        pos = torch.arange(inv.numel(), device=ids.device)
        last = torch.full((uni.numel(),), -1, dtype=torch.long, device=ids.device)
        return last.scatter_reduce(0, inv, pos, reduce="amax", include_self=True)

    def push_update_memory(self, nid, memory, root_nodes, ts, neg_samples=1):
        """memorys.py:190-204: the rows update_memory would write, one per node."""
        if nid is None:
            return
        k = len(root_nodes) // (neg_samples + 2) * 2
        with torch.no_grad():
            nid, memory, ts = nid[:k], memory[:k], ts[:k]
            perm = self._last_rows(_ids(nid, memory.device))
            return nid[perm].to(self.device), memory[perm], ts[perm]

    def update_memory_trans(self, nid, memory, ts):
        """memorys.py:206-210 (ids already distinct)."""
        self._ensure_gpu()
        with torch.no_grad():
            ids = _ids(nid, self.device)
            last, gen = self._tags()
            fastAgg.memory_update_(ids, _as_device(memory, self.device, torch.float32),
                                   _as_device(ts, self.device, torch.float32), self.node_memory,
                                   self.node_memory_ts, last, gen)

    def push_update_mailbox(self, nid, memory, root_nodes, ts, edge_feats, edges=None,
                            uni_node=None, inv_node=None, neg_samples=1):
        """memorys.py:212-253 for deliver_to 'self': (node ids, mails, mail times), one per
        node, the last mail of each."""
        if self.memory_param["deliver_to"] != "self":
            raise NotImplementedError("deliver_to 'neighbors' (APAN) is not built here")
        n = len(root_nodes) // (neg_samples + 2)
        with torch.no_grad():
            dev = memory.device
            roots = _ids(root_nodes, dev)
            src, dst = roots[:n], roots[n:2 * n]
            ms, md = memory[:n], memory[n:2 * n]
            parts_s, parts_d = [ms, md], [md, ms]
            if self.dim_edge_feat > 0:
                ef = _as_device(edge_feats[:n], dev, torch.float32)
                parts_s.append(ef)
                parts_d.append(ef)
            mail = torch.cat([torch.cat(parts_s, 1), torch.cat(parts_d, 1)], 1).reshape(2 * n, -1)
            ids = torch.stack([src, dst], 1).reshape(-1)
            mail_ts = _as_device(ts[:2 * n], dev, torch.float32)
            perm = self._last_rows(ids)
            return ids[perm].to(self.device), mail[perm], mail_ts[perm]

    def update_mailbox_trans(self, nid, mail, mail_ts):
        """memorys.py:255-266 (ids already distinct): slot next_mail_pos of each node."""
        if self.memory_param["mail_combine"] != "last":
            raise NotImplementedError("mail_combine " + str(self.memory_param["mail_combine"]))
        self._ensure_gpu()
        with torch.no_grad():
            ids = _ids(nid, self.device).long()
            pos = self.next_mail_pos[ids]
            self.mailbox[ids, pos] = _as_device(mail, self.device, torch.float32)
            self.mailbox_ts[ids, pos] = _as_device(mail_ts, self.device, torch.float32)
            if self.memory_param["mailbox_size"] > 1:
                if self.update_mail_pos is None:
                    self.next_mail_pos[ids] = torch.remainder(pos + 1, self.memory_param["mailbox_size"])
                else:
                    self.update_mail_pos[ids] = 1


class _CellUpdate(torch.autograd.Function):
    """Time columns + recurrent cell over rows x = [mails | time features]."""

    @staticmethod
    def forward(ctx, rows, mail_w, ts, mem_ts, h, w_ih, w_hh, b_ih, b_hh, tw, tb, gru):
        dt = 0 if tw is None else tw.numel()
        n, m = h.shape
        if dt:
            _timed("time_rows", n * (8 + 4 * dt), fastAgg.time_rows_, rows, mail_w, ts, mem_ts, tw, tb)
        # the input and hidden products on the split-bf16 reduce kernel (torch's GEMM where
        # it does not take the shape), without their biases, which the gate kernel adds
        gi = tgat._rows_mm(rows, w_ih, "cell_proj")
        gh = tgat._rows_mm(h, w_hh, "cell_proj")
        if gru:
            # gi, gh, h read; h' and the [r | z | c | gh_n] workspace written
            hy, saved = _timed("cell_fwd", n * m * 48, fastAgg.gru_fwd, gi, gh, h, b_ih, b_hh)
        else:
            hy = _timed("cell_fwd", n * m * 12, fastAgg.rnn_fwd, gi, gh, b_ih, b_hh)
            saved = hy
        ctx.gru, ctx.mail_w, ctx.dt = gru, mail_w, dt
        ctx.save_for_backward(rows, h, w_ih, w_hh, saved, ts, mem_ts, tw, tb)
        return hy

    @staticmethod
    def backward(ctx, dhy):
        rows, h, w_ih, w_hh, saved, ts, mem_ts, tw, tb = ctx.saved_tensors
        dhy = dhy.contiguous()
        need_h = ctx.needs_input_grad[4]
        n, m = dhy.shape
        if ctx.gru:
            # dhy, workspace, h read; dgi, dgh (and dh) written; the bias sums on the way
            nb = n * m * (48 + (4 if need_h else 0))
            dgi, dgh, dh_direct, d_bih, d_bhh = _timed("cell_bwd", nb, fastAgg.gru_bwd, dhy, saved,
                                                       h, need_h)
        else:
            dgi = dgh = _timed("cell_bwd", n * m * 12, fastAgg.rnn_bwd, dhy, saved)
            d_bih = d_bhh = dgi.sum(0)
            dh_direct = None
        d_wih = _tmm(dgi, rows) if ctx.needs_input_grad[5] else None
        d_whh = _tmm(dgh, h) if ctx.needs_input_grad[6] else None
        d_bih = d_bih if ctx.needs_input_grad[7] else None
        d_bhh = d_bhh if ctx.needs_input_grad[8] else None
        d_tw = d_tb = None
        if ctx.dt and (ctx.needs_input_grad[9] or ctx.needs_input_grad[10]):
            # the time columns' gradient dgi W_ih[:, mail_w:]
            g_time = tgat._rows_mm(dgi, w_ih[:, ctx.mail_w:].t(), "cell_reduce")
            d_tw, d_tb = _timed("time_rows_grad", n * (8 + 4 * ctx.dt), fastAgg.time_rows_grad,
                                g_time, ts, mem_ts, tw, tb)
            d_tw = d_tw.view_as(tw)
        dh = None
        if need_h:
            dh = dgh.mm(w_hh)
            if dh_direct is not None:
                dh = dh + dh_direct
        return None, None, None, None, dh, d_wih, d_whh, d_bih, d_bhh, d_tw, d_tb, None


def _cell_rows(b, mail_w: int, dt: int) -> torch.Tensor:
    """The block's updater rows [n, mail_w + dt] holding the mails in the first mail_w
    columns: the gather's own rows when present, else a copy of srcdata['mem_input']."""
    rows = b.srcdata.get("_mem_rows")
    mi = b.srcdata["mem_input"]
    if (rows is not None and rows.shape == (mi.shape[0], mail_w + dt)
            and mi.data_ptr() == rows.data_ptr() and mi.shape[1] == mail_w):
        return rows
    rows = torch.empty((mi.shape[0], mail_w + dt), dtype=torch.float32, device=mi.device)
    rows[:, :mail_w] = mi
    return rows


class _RecurrentUpdater(torch.nn.Module):
    """Shared forward of GRUMemeoryUpdater / RNNMemeoryUpdater (memorys.py:268-340)."""

    gru = True

    def __init__(self, memory_param, dim_in, dim_hid, dim_time, dim_node_feat):
        super().__init__()
        self.dim_hid = dim_hid
        self.dim_node_feat = dim_node_feat
        self.memory_param = memory_param
        self.dim_time = dim_time
        cell = torch.nn.GRUCell if self.gru else torch.nn.RNNCell
        self.updater = cell(dim_in + dim_time, dim_hid)
        self.last_updated_memory = None
        self.last_updated_ts = None
        self.last_updated_nid = None
        if dim_time > 0:
            self.time_enc = TimeEncode(dim_time)
        if memory_param["combine_node_feature"]:
            if dim_node_feat > 0 and dim_node_feat != dim_hid:
                self.node_feat_map = torch.nn.Linear(dim_node_feat, dim_hid)

    def forward(self, mfg):
        u = self.updater
        for b in mfg:
            mail_w = b.srcdata["mem_input"].shape[1]
            rows = _cell_rows(b, mail_w, self.dim_time)
            ts = b.srcdata["ts"].to(torch.float32).contiguous()
            mem_ts = b.srcdata["mem_ts"].contiguous()
            mem = b.srcdata["mem"].contiguous()
            tw = self.time_enc.w.weight.view(-1) if self.dim_time > 0 else None
            tb = self.time_enc.w.bias if self.dim_time > 0 else None
            updated = _CellUpdate.apply(rows, mail_w, ts, mem_ts, mem, u.weight_ih, u.weight_hh,
                                        u.bias_ih, u.bias_hh, tw, tb, self.gru)
            b.srcdata["mem_input"] = rows
            self.last_updated_ts = b.srcdata["ts"].detach().clone()
            self.last_updated_memory = updated.detach().clone()
            self.last_updated_nid = b.srcdata["ID"].detach().clone()
            if self.memory_param["combine_node_feature"]:
                if self.dim_node_feat > 0:
                    if self.dim_node_feat == self.dim_hid:
                        b.srcdata["h"] = b.srcdata["h"] + updated
                    else:
                        b.srcdata["h"] = updated + self.node_feat_map(b.srcdata["h"])
                else:
                    b.srcdata["h"] = updated


class GRUMemeoryUpdater(_RecurrentUpdater):
    """memorys.py:268-304 (torch.nn.GRUCell over [mails, time features])."""

    gru = True


class RNNMemeoryUpdater(_RecurrentUpdater):
    """memorys.py:306-340 (torch.nn.RNNCell, tanh)."""

    gru = False
