"""Composed CPU oracle of the expert-FFN layer step (test infrastructure).

The layer (the reference's e2e_bench.py:56-134 on MXFP8) is checked stage by
stage.  Every GEMM output that feeds a later stage (h = [gate | up], dA) comes
from the library and is itself held against the oracle's dequantise + float64
matmul; everything downstream of it (SwiGLU forward and backward, every cast,
the next GEMM) is recomputed by the oracle from those library values, so an
error in any one stage shows up at that stage, at the 1e-2 bound of
assert_close_to_oracle, not as drift through the layer.

Outputs are sampled: rows of y and dX, and (output feature, input feature)
pairs of both weight gradients for every expert.
"""
from __future__ import annotations

import numpy as np
import torch

from mxfp8gg import ops
from oracle import oracle as O
from tests._helpers import assert_close_to_oracle, bits, u8


def _fwd_rows(a_q, a_s, w_q, w_s, gids):
    """Rows of a grouped forward: row i uses expert gids[i]; a_q / a_s numpy
    [R, K] / [R, K/32]; w_q / w_s device tensors [E, N, K] / [E, N, K/32]."""
    out = np.empty((a_q.shape[0], w_q.shape[1]))
    for g in np.unique(gids):
        sel = gids == g
        w = O.dequant(u8(w_q[int(g)]), u8(w_s[int(g)]))
        out[sel] = O.dequant(a_q[sel], a_s[sel]) @ w.T
    return out


def check_layer(x, wgu, wd, dy, sizes, rows, n_feat, f_feat, m_feat, k_feat, got):
    """Hold the library's layer step `got` = dict(y, dx, dwgu, dwd) against the
    composed oracle.

    x bf16 [M, H]; wgu [E, 2F, H]; wd [E, H, F]; dy [M, H]; sizes [E];
    rows: sampled token rows (sorted, inside the groups); n_feat, f_feat:
    sampled (output, input) features of dW_down [E, H, F]; m_feat, k_feat: of
    dW_gate_up [E, 2F, H]."""
    E, F2, H = wgu.shape
    F = F2 // 2
    M = x.shape[0]
    ends_np = np.cumsum(np.asarray(sizes, dtype=np.int64)).astype(np.int32)
    ends = torch.from_numpy(ends_np).to(x.device)
    rows = np.asarray(rows)
    ri = torch.from_numpy(rows).to(x.device)
    gids = np.searchsorted(ends_np, rows, side="right")

    # ---- forward ---------------------------------------------------------
    xq, xs = ops.to_mxfp8_dim0(x)
    rq, rs = O.quant_dim0(bits(x[ri]))
    assert np.array_equal(u8(xq[ri]), rq) and np.array_equal(u8(xs[ri]), rs), "cast of X"
    (wq, ws), (wgt, wgts) = ops.quant_weight_dual(wgu)
    (wdq, wds), (wdt, wdts) = ops.quant_weight_dual(wd)
    h = ops.grouped_mm(xq, wq, ends, xs, ws)
    assert_close_to_oracle(h[ri], _fwd_rows(rq, rs, wq, ws, gids))
    hb = bits(h[ri])
    a_bits = O.swiglu_fwd(hb[:, :F], hb[:, F:])
    aq_ref, as_ref = O.quant_dim0(a_bits)
    assert_close_to_oracle(got["y"][ri], _fwd_rows(aq_ref, as_ref, wdq, wds, gids))

    # ---- backward: dA = dY . W_down, SwiGLU backward, dX = dH . W_gate_up -
    dyq, dys = ops.to_mxfp8_dim0(dy)
    dq_ref, ds_ref = O.quant_dim0(bits(dy[ri]))
    assert np.array_equal(u8(dyq[ri]), dq_ref) and np.array_equal(u8(dys[ri]), ds_ref), "cast of dY"
    da = ops.grouped_mm(dyq, wdt, ends, dys, wdts)
    assert_close_to_oracle(da[ri], _fwd_rows(dq_ref, ds_ref, wdt, wdts, gids))
    _, dg, du = O.swiglu_bwd(hb[:, :F], hb[:, F:], bits(da[ri]))
    dhq_ref, dhs_ref = O.quant_dim0(np.concatenate([dg, du], axis=1))
    assert_close_to_oracle(got["dx"][ri], _fwd_rows(dhq_ref, dhs_ref, wgt, wgts, gids))

    # ---- weight gradients: token-axis casts per expert, then dY^T a / dH^T X
    cap = ops.padded_token_capacity(M, E)
    n_feat, f_feat = np.asarray(n_feat), np.asarray(f_feat)
    m_feat, k_feat = np.asarray(m_feat), np.asarray(k_feat)
    ni = torch.from_numpy(n_feat).to(x.device)
    fi = torch.from_numpy(f_feat).to(x.device)
    h_g = bits(h[:, torch.from_numpy(f_feat).to(x.device)])
    h_u = bits(h[:, torch.from_numpy(f_feat + F).to(x.device)])
    a_cols = O.swiglu_fwd(h_g, h_u)                                # [M, |f|]
    aqt, ast, pad = O.quant_dim1(a_cols, ends_np, cap)
    dyqt, dyst, pad2 = O.quant_dim1(bits(dy[:, ni]), ends_np, cap)
    assert np.array_equal(pad, pad2)
    ref = O.grouped_wgrad(dyqt, dyst, aqt, ast, pad)               # [E, |n|, |f|]
    got_d = got["dwd"][:, ni][:, :, fi]
    for e in range(E):
        if sizes[e]:
            assert_close_to_oracle(got_d[e], ref[e])
        else:
            assert torch.all(got_d[e] == 0)

    j = m_feat % F                                                 # the SwiGLU column
    ji = torch.from_numpy(j).to(x.device)
    _, dg_c, du_c = O.swiglu_bwd(bits(h[:, ji]), bits(h[:, ji + F]), bits(da[:, ji]))
    dh_cols = np.where((m_feat < F)[None, :], dg_c, du_c)          # [M, |m|]
    dhqt, dhst, _ = O.quant_dim1(dh_cols, ends_np, cap)
    ki = torch.from_numpy(k_feat).to(x.device)
    xqt, xst, _ = O.quant_dim1(bits(x[:, ki]), ends_np, cap)
    ref = O.grouped_wgrad(dhqt, dhst, xqt, xst, pad)               # [E, |m|, |k|]
    got_g = got["dwgu"][:, torch.from_numpy(m_feat).to(x.device)][:, :, ki]
    for e in range(E):
        if sizes[e]:
            assert_close_to_oracle(got_g[e], ref[e])
        else:
            assert torch.all(got_g[e] == 0)
