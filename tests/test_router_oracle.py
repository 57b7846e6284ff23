"""CPU pins of the router oracle (the reference engine's routing,
kernel/cpp-engine-mxfp4/routed.cu:124-208 and runtime/dsv4_engine_mxfp4.py:363-370):
the score against torch and closed forms, the selection against torch.topk and
the scalar C restatement (first strictly larger score wins), the weights
against closed forms, the router GEMV against the fp64 C oracle and a one-hot
column, and planted mistakes that these pins must catch."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import c_oracle as co
from oracle import mx
from runtime import synth


def _ulp_diff(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


def test_sqrt_softplus_against_torch_and_closed_forms():
    l = synth.gating_logits(51, 8, 256) * np.float32(4.0)
    l = np.concatenate([l.reshape(-1), np.array([0, 1e-8, -1e-8, 15, 25, 40, 88, -30, -87, -100], np.float32)])
    s = mx.sqrt_softplus(l)
    t = torch.sqrt(torch.nn.functional.softplus(torch.from_numpy(l))).numpy()
    assert np.max(_ulp_diff(s, t)) <= 2
    assert s[np.where(l == 0)[0][0]] == np.float32(math.sqrt(math.log(2.0)))
    big = np.array([30.0, 60.0, 1e6], np.float32)
    assert np.array_equal(mx.sqrt_softplus(big), np.sqrt(big))
    special = mx.sqrt_softplus(np.array([-np.inf, np.inf, np.nan], np.float32))
    assert special[0] == 0.0 and special[1] == np.inf and np.isnan(special[2])
    # fp64 closed form over a grid (the score is monotone increasing)
    g = np.linspace(-20, 20, 4001).astype(np.float32)
    ref = np.sqrt(np.logaddexp(0.0, g.astype(np.float64)))
    assert np.max(np.abs(mx.sqrt_softplus(g) - ref) / ref) < 3e-7
    assert np.all(np.diff(mx.sqrt_softplus(g)) >= 0)


def test_selection_matches_torch_topk_and_c_restatement():
    logits = synth.gating_logits(52, 32, 256) * np.float32(2.0)
    ids, w = mx.route_sqrt_softplus_topk(logits, 6)
    tv, ti = torch.topk(torch.sqrt(torch.nn.functional.softplus(torch.from_numpy(logits))), 6, dim=-1)
    assert np.array_equal(ids, ti.numpy().astype(np.int32))
    cids, cw, found = co.route_sqrt_softplus(logits, 6, 1.5)
    assert np.array_equal(ids, cids) and np.all(found == 6)
    assert np.array_equal(w, cw)


def test_selection_ties_nan_and_infinities():
    rows = [
        np.zeros(16, np.float32),                                       # all equal: 0..k-1
        np.array([1, 3, 3, 2, 3, 0, 3, 1] * 2, np.float32),             # ties at the top
        np.array([np.nan, 2, np.nan, 1, -np.inf, 5, np.inf, 0] * 2, np.float32),
        np.array([-np.inf] * 12 + [1, np.nan, -np.inf, 2], np.float32),
        np.array([-50, -60, -45, -45, -70, -80, -55, -45] * 2, np.float32),  # tiny scores
    ]
    for k in (1, 6, 8):
        for r in rows:
            ids, w = mx.route_sqrt_softplus_topk(r[None, :], k)
            cids, cw, found = co.route_sqrt_softplus(r[None, :], k, 1.5)
            assert np.array_equal(ids, cids), (r, k, ids, cids)
            if found[0] == k:
                assert np.array_equal(w, cw, equal_nan=True)
    assert mx.route_sqrt_softplus_topk(rows[0][None, :], 4)[0].tolist() == [[0, 1, 2, 3]]
    assert mx.route_sqrt_softplus_topk(rows[1][None, :], 3)[0].tolist() == [[1, 2, 4]]
    # +inf first, NaN never before a number
    ids = mx.route_sqrt_softplus_topk(rows[2][None, :], 8)[0][0].tolist()
    assert ids[:2] == [6, 14] and all(not np.isnan(rows[2][i]) for i in ids)


def test_weights_closed_forms():
    logits = synth.gating_logits(53, 16, 256)
    ids, w = mx.route_sqrt_softplus_topk(logits, 6, 1.5)
    s = mx.sqrt_softplus(logits).astype(np.float64)
    sel = np.take_along_axis(s, ids.astype(np.int64), axis=1)
    S = sel.sum(1)
    assert np.allclose(w.astype(np.float64).sum(1), 1.5 * S / (S + 1e-20), rtol=1e-6)
    assert np.allclose(w[:, 1:] / w[:, :1], sel[:, 1:] / sel[:, :1], rtol=1e-6)
    assert np.all(np.diff(w, axis=1) <= 0)                        # descending with the scores
    w2 = mx.route_sqrt_softplus_topk(logits, 6, 2.5)[1]
    assert np.allclose(w2 / w, 2.5 / 1.5, rtol=1e-6)
    # all-(-inf) logits: scores 0, weights 0 / 1e-20 = 0
    ids0, w0 = mx.route_sqrt_softplus_topk(np.full((1, 8), -np.inf, np.float32), 3)
    assert ids0.tolist() == [[0, 1, 2]] and np.all(w0 == 0)


def test_router_logits_against_c_oracle_and_one_hot():
    x = synth.normal_bf16(54, (3, 1000))
    wg = synth.normal_bf16(55, (40, 1000), 0.0, 0.02)
    ref = co.router_logits(x, wg)
    got = mx.router_logits(x, wg)
    assert np.array_equal(got, ref)
    one = np.zeros((1, 1000), np.uint16)
    one[0, 123] = 0x3F80                                         # bf16 1.0
    col = mx.router_logits(one, wg)[0]
    assert np.array_equal(col, mx.bf16_to_f32(wg[:, 123]))
    # against torch's fp32 GEMV of the reference's Python engine (a few ulps of sum |W x|)
    tx = torch.from_numpy(mx.bf16_to_f32(x))
    tw = torch.from_numpy(mx.bf16_to_f32(wg))
    t = torch.nn.functional.linear(tx, tw).numpy()
    bound = (np.abs(mx.bf16_to_f32(x)) @ np.abs(mx.bf16_to_f32(wg)).T) * 1e-5
    assert np.all(np.abs(t - got) <= bound)


def test_planted_mistakes_are_caught():
    """Plausible mistakes in a copy of the router oracle fail the pins above."""
    logits = synth.gating_logits(56, 8, 256)
    ids, w = mx.route_sqrt_softplus_topk(logits, 6, 1.5)
    cids, cw, _ = co.route_sqrt_softplus(logits, 6, 1.5)
    # (a) scores without the square root: the weight ratios change
    sp = np.maximum(logits, 0) + np.log1p(np.exp(-np.abs(logits)))
    sel = np.take_along_axis(sp, ids.astype(np.int64), axis=1).astype(np.float64)
    bad_a = (sel / sel.sum(1, keepdims=True) * 1.5).astype(np.float32)
    assert not np.allclose(bad_a, cw, rtol=1e-4)
    # (b) the routed scale dropped: the weights sum to 1, not 1.5
    assert not np.allclose(w / 1.5, cw, rtol=1e-4)
    # (c) ties to the higher index
    tie = np.array([[1, 3, 3, 2, 3, 0, 3, 1]], np.float32)
    bad_c = np.argsort(-mx.sqrt_softplus(tie)[:, ::-1], axis=1, kind="stable")[:, :2]
    bad_c = (tie.shape[1] - 1 - bad_c).astype(np.int32)
    assert not np.array_equal(bad_c, co.route_sqrt_softplus(tie, 2, 1.5)[0])
    assert np.array_equal(ids, cids)
