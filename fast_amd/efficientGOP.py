"""Flag manager and autograd wrappers of FAST's operator layer, bound to the gfx950 kernels.

Mirrors the interface of the reference's ``fast_util/efficientGOP.py`` (efficientGOP.py:6-136
for the live wrappers, 141-289 for the deprecated ones): the global ``fm`` with
``init_gop(fast_agg, fast_esm, csr_out)``, ``ESM_Function_TGAT``, ``MA_Function_TGAT``,
``unique2indptr``, ``FUSED_TGAT``, ``FAST_DROP`` and ``FAST_QKV``, with the same
``apply`` argument order, so the reference ``layers.py`` can import this module in place of
its own. Differences, all deliberate:
  * ``ESM_Function_TGAT`` softmaxes every head of its input unless ``num_heads`` is given
    (the reference always passed 2, efficientGOP.py:68);
  * the kernels behind the wrappers aggregate every edge and give the exact transpose in
    backward (see fastAgg);
  * ``FUSED_TGAT.backward`` applies the LeakyReLU derivative to the kernel's softmax-input
    gradient, so the returned gradient is the one of its pre-activation input.
"""
from __future__ import annotations

import torch

from . import fastAgg


class forwardManager:
    """Global operator flags and launch parameters (efficientGOP.py:6-38)."""

    def __init__(self):
        self.fastAggFlag = 0
        self.fastESMFlag = 0
        self.CSR_OUT = 0
        self.reduceSize = 16
        self.node_num_per_block = 1
        self.aggFeat = 1
        self.aggNodePB = 1
        self.fastKQV = 0
        self.fastTIME = 0
        self.fastDrop = 0
        self.cntE = []        # per-layer int32 indptr from the sampler (train.py:339-343)
        self.layerAllNum = 1  # set by the model (modules.py:56)

    def init_gop(self, fast_agg=0, fast_esm=0, csr_out=0):
        self.fastAggFlag = fast_agg
        self.fastESMFlag = fast_esm
        self.CSR_OUT = csr_out
        # Launch parameters chosen per method in the reference; the gfx950 kernels accept
        # them for signature compatibility and pick their own launch shapes.
        if fast_esm == 2:
            self.reduceSize = 16
            self.node_num_per_block = max(1, int(1024 / self.reduceSize / 2))
        elif fast_esm == 1:
            self.node_num_per_block = 512
            self.reduceSize = 16
        if fast_agg == 2:
            self.aggNodePB = 8
            self.aggFeat = 32
        elif fast_agg == 1:
            self.aggNodePB = 8
            self.aggFeat = 128


fm = forwardManager()


class ESM_Function_TGAT(torch.autograd.Function):
    """Segmented edge softmax over CSR segments (efficientGOP.py:66-95)."""

    @staticmethod
    def forward(ctx, dst_eid, src_eid, input_feat, node_num, num_heads=None):
        indptr, indices = dst_eid, src_eid
        heads = input_feat.size(1) if num_heads is None else int(num_heads)
        if fm.fastESMFlag == 1:
            out = fastAgg.forward_edge_softmax(indptr, indices, input_feat,
                                               fm.node_num_per_block, heads)[0]
        elif fm.fastESMFlag == 2:
            out = fastAgg.forward_csr_edge_softmax(indptr, indices, input_feat,
                                                   fm.node_num_per_block, fm.reduceSize)[0]
        else:
            raise ValueError("fastESMFlag must be 1 or 2")
        ctx.num_heads = heads
        ctx.save_for_backward(indptr, indices, out)
        return out

    @staticmethod
    def backward(ctx, d_out):
        indptr, indices, out = ctx.saved_tensors
        d_out = d_out.contiguous()
        out = out.contiguous()
        if fm.fastESMFlag == 1:
            d_x = fastAgg.backward_edge_softmax(indptr, indices, d_out, out,
                                                fm.node_num_per_block, ctx.num_heads)[0]
        elif fm.fastESMFlag == 2:
            d_x = fastAgg.backward_csr_edge_softmax(indptr, indices, d_out, out,
                                                    fm.node_num_per_block, fm.reduceSize)[0]
        else:
            raise ValueError("fastESMFlag must be 1 or 2")
        return None, None, d_x, None, None


class MA_Function_TGAT(torch.autograd.Function):
    """Sum aggregation of source rows into destinations (efficientGOP.py:97-131).

    ``src_edge`` holds the destination id of every edge and ``dst_edge`` its source id,
    as at the reference call sites (layers.py:210-222).
    """

    @staticmethod
    def forward(ctx, src_edge, dst_edge, input_feat, num_dst_nodes, neighbor_num=10,
                num_heads=2, densePtr=None, denseInd=None):
        if fm.fastAggFlag == 2:
            out = fastAgg.forward_tgat_shd(densePtr, denseInd, src_edge, dst_edge, input_feat,
                                           num_dst_nodes, fm.aggNodePB, fm.aggFeat)[0]
            ctx.save_for_backward(src_edge, dst_edge, densePtr, denseInd)
        elif fm.fastAggFlag == 1:
            out = fastAgg.forward_tgat(src_edge, dst_edge, input_feat, num_dst_nodes,
                                       fm.aggNodePB, fm.aggFeat)[0]
            ctx.save_for_backward(src_edge, dst_edge)
        else:
            raise ValueError("fastAggFlag must be 1 or 2")
        ctx.src_nodes = input_feat.size(0)
        ctx.num_heads = num_heads
        ctx.neighbor_num = neighbor_num
        return out

    @staticmethod
    def backward(ctx, d_out):
        d_out = d_out.contiguous()
        if fm.fastAggFlag == 2:
            src_edge, dst_edge, densePtr, denseInd = ctx.saved_tensors
            d_x = fastAgg.backward_tgat_shd(densePtr, denseInd, src_edge, dst_edge, d_out,
                                            ctx.src_nodes, fm.aggNodePB, fm.aggFeat)[0]
        elif fm.fastAggFlag == 1:
            src_edge, dst_edge = ctx.saved_tensors
            d_x = fastAgg.backward_tgat(src_edge, dst_edge, d_out, ctx.src_nodes,
                                        fm.aggNodePB, fm.aggFeat)[0]
        else:
            raise ValueError("fastAggFlag must be 1 or 2")
        return None, None, d_x, None, None, None, None, None


def unique2indptr(dstID, dstNum):
    """int32 CSR offsets over the non-empty destinations of ``dstID`` (efficientGOP.py:133-136)."""
    _, deg = torch.unique(dstID, return_counts=True)
    return fastAgg.exclusive_sum(deg.int())


class FUSED_TGAT(torch.autograd.Function):
    """LeakyReLU + softmax + dropout + aggregation in one operator (efficientGOP.py:234-264)."""

    @staticmethod
    def forward(ctx, input_feat, Vval, indptr, indices, dst_eid, src_eid, node_num_dst,
                node_num_src, num_heads=2, negative_slope=0.2, attn_drop=0.1):
        out, attn, mask = fastAgg.forward_fused_attn(input_feat, Vval.contiguous(), indptr,
                                                     indices, dst_eid, src_eid, node_num_dst,
                                                     num_heads, negative_slope, attn_drop)
        ctx.node_num = node_num_src
        ctx.num_heads = num_heads
        ctx.negative_slope = negative_slope
        ctx.attn_drop = attn_drop
        ctx.save_for_backward(input_feat, Vval, attn, mask, indptr, indices, dst_eid, src_eid)
        return out

    @staticmethod
    def backward(ctx, d_out):
        input_feat, Vval, attn, mask, indptr, indices, dst_eid, src_eid = ctx.saved_tensors
        d_act, grad_V = fastAgg.backward_fused_attn(
            d_out.contiguous(), Vval.contiguous(), attn, mask, indptr, indices, dst_eid, src_eid,
            ctx.node_num, ctx.num_heads, ctx.negative_slope, ctx.attn_drop)
        slope = torch.full_like(input_feat, ctx.negative_slope)
        d_x = d_act * torch.where(input_feat > 0, torch.ones_like(input_feat), slope)
        return d_x, grad_V.view_as(Vval), None, None, None, None, None, None, None, None, None


class FAST_DROP(torch.autograd.Function):
    """V*att followed by prepending N zero rows (efficientGOP.py:266-289)."""

    @staticmethod
    def forward(ctx, attn, Vval, node_num):
        with torch.no_grad():
            v = (Vval * attn[:, :, None]).reshape(Vval.shape[0], -1)
            out = torch.cat([v.new_zeros((node_num, v.shape[1])), v], dim=0)
        ctx.save_for_backward(Vval, attn)
        ctx.node_num = node_num
        return out

    @staticmethod
    def backward(ctx, d_out):
        Vval, attn = ctx.saved_tensors
        d = d_out.contiguous()[ctx.node_num:].reshape(Vval.shape)
        return (d * Vval).sum(-1), d * attn[:, :, None], None


class FAST_QKV(torch.autograd.Function):
    """Q/K/V projections of the concatenated inputs with a hand-written backward
    (efficientGOP.py:141-231). Returns per-edge Q, K, V. With ``fm.fastTIME`` the time
    inputs are the encoder's pre-cosine arguments and the cosine is applied here."""

    @staticmethod
    def forward(ctx, w_q, w_k, w_v, b_q, b_k, b_v, nFeat, eFeat, eid, timeFeat, zeroFeat,
                num_nodes, dim_out=100):
        fast_time = bool(fm.fastTIME)
        with torch.no_grad():
            tf = torch.cos(timeFeat) if fast_time else timeFeat
            zf = torch.cos(zeroFeat) if fast_time else zeroFeat
            if zf.shape[0] != num_nodes:
                zf = zf.expand(num_nodes, -1)
            q_in = torch.cat([nFeat[:num_nodes], zf], dim=1)
            kv_in = torch.cat([nFeat[num_nodes:], eFeat, tf], dim=1)
            Q = torch.nn.functional.linear(q_in, w_q, b_q)[eid]
            K = torch.nn.functional.linear(kv_in, w_k, b_k)
            V = torch.nn.functional.linear(kv_in, w_v, b_v)
        ctx.save_for_backward(w_q, w_k, w_v, q_in, kv_in, timeFeat, zeroFeat, eid)
        ctx.num_nodes = num_nodes
        ctx.fast_time = fast_time
        ctx.split = nFeat.shape[1] + eFeat.shape[1]
        ctx.nsplit = nFeat.shape[1]
        return Q, K, V

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        w_q, w_k, w_v, q_in, kv_in, timeFeat, zeroFeat, eid = ctx.saved_tensors
        with torch.no_grad():
            gq = torch.zeros(ctx.num_nodes, grad_q.shape[1], dtype=grad_q.dtype,
                             device=grad_q.device).index_add_(0, eid, grad_q.contiguous())
            gk, gv = grad_k.contiguous(), grad_v.contiguous()
            d_wq, d_bq = gq.t() @ q_in, gq.sum(0)
            d_wk, d_bk = gk.t() @ kv_in, gk.sum(0)
            d_wv, d_bv = gv.t() @ kv_in, gv.sum(0)
            d_zero = (gq @ w_q)[:, ctx.nsplit:]
            d_time = gk @ w_k[:, ctx.split:] + gv @ w_v[:, ctx.split:]
            if ctx.fast_time:
                d_zero = d_zero * (-torch.sin(zeroFeat))
                d_time = d_time * (-torch.sin(timeFeat))
            if zeroFeat.shape[0] != ctx.num_nodes:
                d_zero = d_zero.sum(0, keepdim=True)
        return (d_wq, d_wk, d_wv, d_bq, d_bk, d_bv, None, None, None, d_time, d_zero, None, None)
