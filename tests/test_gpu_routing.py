"""GPU parity of the routed paths at the configuration's shapes and of the
reference engine's routing on the device, through the C ABI, against the CPU
oracle.

Covered here: every one-token stage-A variant at K = 4096 (routing tables
given, caller's ids, gated) on the configuration's 256 experts; the general
one-token stage B (more than 8 routed slots: the drop-in with 16 to 256
experts, top-16 layers); a three-layer chained decode with Zipf routing; the
routing outputs with one pointer given; the prefill decode bit for bit; the
router GEMV, the sqrt-softplus scoring and the routed dispatch.
Bar: outputs max rel err <= 1e-2 and cosine >= 0.9999 against the oracle;
ids bit-exact; weights to float rounding.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import mx
from runtime import moe, synth
from runtime import mxfp4_grouped_gemv_binding as gb
from tests.gpu_util import announce, assert_close, dev_bf16, dev_f32, dev_u8, host_bits

pytestmark = pytest.mark.gpu

E3, K3, H3, O3 = 256, 4096, 2048, 4096      # configuration 3 shapes


def _host_expert_fn(weights):
    cache = {}

    def fn(e):
        if e not in cache:
            cache[e] = tuple((m["packed"][e].cpu().numpy(), m["scale"][e].cpu().numpy())
                             for m in (weights.W1, weights.W3, weights.W2))
        return cache[e]

    return fn


@pytest.fixture(scope="module")
def cfg3_layer(device):
    w = moe.make_moe_weights(12000, E3, K3, H3, O3, device)
    yield w
    del w
    torch.cuda.empty_cache()


# --------------------------------------------------------------- decoding --

def test_prefill_dequant_exhaustive_bit_exact(device):
    """The prefill GEMMs' decode: every packed byte under every scale byte
    (0 -> 2^-127, 0xFF -> 0, as the decode path and the reference)."""
    announce("mxfp4_moe_prefill_dequant_bf16 exhaustive 256x512")
    packed = np.tile(np.arange(256, dtype=np.uint8), (256, 1))
    scale = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    got = host_bits(gb.prefill_dequant(dev_u8(packed, device), dev_u8(scale, device)))
    assert np.array_equal(got, mx.mxfp4_dequant_bf16(packed, scale, kernel_convention=True))


# ------------------------------------------- one token at the config shapes --

def test_one_token_stage_a_variants_at_config_shapes(device, cfg3_layer):
    """K = 4096, 256 experts, top-8: stage A with the routing tables given
    (build_routing, then mxfp4_moe_swiglu), with the caller's ids (two-launch
    mxfp4_moe_grouped_gemv) and gated (mxfp4_moe_layer) give the same bits and
    match the oracle."""
    w = cfg3_layer
    x = synth.normal_bf16(12100, (1, K3))
    logits = synth.gating_logits(12101, 1, E3)
    ids, wt = mx.route_sigmoid_topk(logits, 8)
    xd, idd, wd = dev_bf16(x, device), torch.from_numpy(ids).to(device), dev_f32(wt, device)
    announce("T=1 K=4096 E=256: tables given (moe_swiglu_t1_kernel GATE=0)")
    st = gb.MoEStages(w.W1, w.W3, w.W2, 1, 8, device)
    st.build_routing(idd, wd)
    st.swiglu(xd)
    tables = host_bits(st.down(torch.empty(1, O3, dtype=torch.bfloat16, device=device)))
    announce("T=1 K=4096 E=256: caller's ids (GATE=2)")
    ids_path = host_bits(gb.mxfp4_moe_grouped_gemv(xd, w.W1, w.W3, w.W2, idd, wd))
    announce("T=1 K=4096 E=256: gated (GATE=1)")
    gated = host_bits(gb.mxfp4_moe_layer(xd, dev_f32(logits, device), w.W1, w.W3, w.W2, 8))
    assert np.array_equal(ids_path, tables)
    ref = mx.moe_layer(x, _host_expert_fn(w), ids, wt, O3)
    assert_close(tables, ref, "T=1 tables-given path vs oracle")
    # the gated kernel computes its own weights (float sigmoid); same ids
    assert_close(gated, ref, "T=1 gated path vs oracle")


def test_moe_layer_routing_outputs_one_pointer(device):
    """ids_out and weights_out may each be given alone (one token: published
    by stage A; two tokens: by the routing kernel)."""
    E, K, H, O, k = 64, 2048, 256, 256, 8
    w = moe.make_moe_weights(12200, E, K, H, O, device)
    for T in (1, 2):
        announce(f"mxfp4_moe_layer T={T}: ids_out only, then weights_out only")
        x = dev_bf16(synth.normal_bf16(12210 + T, (T, K)), device)
        logits = synth.gating_logits(12220 + T, T, E)
        rids, rw = mx.route_sigmoid_topk(logits, k)
        ld = dev_f32(logits, device)
        ids = torch.full((T, k), -7, dtype=torch.int32, device=device)
        a = host_bits(gb.mxfp4_moe_layer(x, ld, w.W1, w.W3, w.W2, k, ids_out=ids))
        assert np.array_equal(ids.cpu().numpy(), rids)
        wo = torch.full((T, k), -7.0, dtype=torch.float32, device=device)
        b = host_bits(gb.mxfp4_moe_layer(x, ld, w.W1, w.W3, w.W2, k, weights_out=wo))
        assert np.allclose(wo.cpu().numpy(), rw, rtol=1e-5, atol=1e-6)
        assert np.array_equal(a, b)


# ------------------------------------- more than 8 routed slots per token --

@pytest.mark.parametrize("n_exp,K,H,O", [(16, 4096, 2048, 4096), (64, 2048, 2048, 1024),
                                         (256, 1024, 2048, 128)])
def test_grouped_dropin_many_experts(device, n_exp, K, H, O):
    """The drop-in with n_exp > 8 at hidden 2048: stage B takes the general
    kernel (more slots than waves)."""
    announce(f"mxfp4_grouped_gemv_topk n_exp={n_exp} K={K} H={H} O={O}")
    w = moe.make_moe_weights(12300 + n_exp, n_exp, K, H, O, device)
    x = synth.normal_bf16(12310 + n_exp, (K,))
    r = synth.normal_f64(12320 + n_exp, 0, n_exp)
    r = 1 / (1 + np.exp(-r))
    r = (r / r.sum()).astype(np.float32)
    out = host_bits(gb.mxfp4_grouped_gemv(w.W1, w.W3, w.W2, None, dev_bf16(x, device), dev_f32(r, device)))
    fn = _host_expert_fn(w)
    ids = np.arange(n_exp, dtype=np.int32)[None, :]
    ref = mx.moe_layer(x, fn, ids, r[None, :], O)
    assert_close(out, ref[0], f"drop-in n_exp={n_exp}")
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 4])
def test_moe_hidden_at_cap(device, T):
    """hidden = 4096, the grouped path's cap: stage B with two MX blocks per
    lane (the one-token kernel at T = 1, the general kernel at T = 4), through
    the expert-indexed entry and the gated layer, and the drop-in with 8
    experts, against the oracle."""
    E, K, H, O, k = 16, 2048, 4096, 512, 8
    announce(f"mxfp4 hidden 4096 T={T} E={E} K={K} O={O}")
    w = moe.make_moe_weights(12600 + T, E, K, H, O, device)
    x = synth.normal_bf16(12610 + T, (T, K))
    logits = synth.gating_logits(12620 + T, T, E)
    ids, wt = mx.route_sigmoid_topk(logits, k)
    xd = dev_bf16(x, device)
    fn = _host_expert_fn(w)
    ref = mx.moe_layer(x, fn, ids, wt, O, n_experts=E)
    idp = host_bits(gb.mxfp4_moe_grouped_gemv(xd, w.W1, w.W3, w.W2, torch.from_numpy(ids).to(device),
                                              dev_f32(wt, device)))
    assert_close(idp, ref, f"hidden 4096 ids path T={T}")
    gated = host_bits(gb.mxfp4_moe_layer(xd, dev_f32(logits, device), w.W1, w.W3, w.W2, k))
    assert_close(gated, ref, f"hidden 4096 gated layer T={T}")
    if T == 1:
        sub = {m: {"packed": getattr(w, m)["packed"][:8], "scale": getattr(w, m)["scale"][:8]}
               for m in ("W1", "W3", "W2")}
        r = np.linspace(0.05, 0.2, 8).astype(np.float32)
        out = host_bits(gb.mxfp4_grouped_gemv(sub["W1"], sub["W3"], sub["W2"], None, xd[0], dev_f32(r, device)))
        ref8 = mx.moe_layer(x, fn, np.arange(8, dtype=np.int32)[None, :], r[None, :], O)
        assert_close(out, ref8[0], "hidden 4096 drop-in n_exp=8")
    del w
    torch.cuda.empty_cache()


def test_moe_layer_top16_one_token(device):
    """One token, top-16 of 64 experts at hidden 2048: 16 routed slots, the
    general one-token stage B, through the gated and the ids paths."""
    E, K, H, O, k = 64, 2048, 2048, 512, 16
    announce(f"mxfp4_moe_layer / grouped T=1 top-{k} E={E} K={K} H={H} O={O}")
    w = moe.make_moe_weights(12400, E, K, H, O, device)
    x = synth.normal_bf16(12401, (1, K))
    logits = synth.gating_logits(12402, 1, E)
    ids, wt = mx.route_sigmoid_topk(logits, k)
    gated = host_bits(gb.mxfp4_moe_layer(dev_bf16(x, device), dev_f32(logits, device), w.W1, w.W3, w.W2, k))
    idp = host_bits(gb.mxfp4_moe_grouped_gemv(dev_bf16(x, device), w.W1, w.W3, w.W2,
                                              torch.from_numpy(ids).to(device), dev_f32(wt, device)))
    ref = mx.moe_layer(x, _host_expert_fn(w), ids, wt, O)
    assert_close(gated, ref, "top-16 gated")
    assert_close(idp, ref, "top-16 ids path")
    del w
    torch.cuda.empty_cache()


# ------------------------------------------------------ chained decode -----

def test_chained_decode_three_layers(device):
    """Three configuration-3 layers in sequence, layer l's output the input of
    layer l+1, with Zipf(1.1) routing given as ids (the decode loop of the
    reference engine, kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:742-845,
    calling routed.cu:479-491 once per layer). Each layer is checked against the
    oracle on the same input, and the final output against the oracle's own
    three-layer chain."""
    L = 3
    layers = [moe.make_moe_weights(12500 + 100 * l, E3, K3, H3, O3, device) for l in range(L)]
    mods = [moe.RoutedMoELayer(w, topk=8, max_tokens=1, check=True) for w in layers]
    routing = [synth.zipf_routing(12600, 1, E3, 8, 1.1, layer=l) for l in range(L)]
    x0 = synth.normal_bf16(12601, (1, K3))
    xd = dev_bf16(x0, device)
    x_ref = x0
    for l in range(L):
        ids, wt = routing[l]
        announce(f"chained decode layer {l}: ids {ids[0].tolist()}")
        out = mods[l].forward(xd, ids=torch.from_numpy(ids).to(device), weights=dev_f32(wt, device))
        got = host_bits(out)
        fn = _host_expert_fn(layers[l])
        assert_close(got, mx.moe_layer(host_bits(xd), fn, ids, wt, O3), f"layer {l} on the device's input")
        x_ref = mx.moe_layer(x_ref, fn, ids, wt, O3)
        xd = out.clone()
    assert_close(host_bits(xd), x_ref, "three-layer chain vs the oracle's chain")
    del mods, layers
    torch.cuda.empty_cache()


def test_chained_decode_graph_replays_match_eager(device):
    """Config 4's timed form: three configuration-3 layers chained on the ids
    path (forward(ids=...): stage A forms the slots from the caller's ids,
    two launches per layer), captured in one HIP graph, as bench.py times the
    43-layer sweep (the reference engine's decode loop,
    kernel/cpp-engine-mxfp4/dsv4_engine_mxfp4_wire.cu:742-845, captured and
    replayed as in graph.cu:118,187). Every replay, with eager work of other
    routings and inputs between replays, must give the eager chain's bits,
    and the last layer's output must match the oracle's own three-layer
    chain."""
    L = 3
    layers = [moe.make_moe_weights(12700 + 100 * l, E3, K3, H3, O3, device) for l in range(L)]
    mods = [moe.RoutedMoELayer(w, topk=8, max_tokens=1, check=False) for w in layers]
    routing = [synth.zipf_routing(12800, 2, E3, 8, 1.1, layer=l) for l in range(L)]
    ids_d = [torch.from_numpy(r[0]).to(device) for r in routing]
    w_d = [dev_f32(r[1], device) for r in routing]
    x0 = synth.normal_bf16(12801, (1, K3))
    x1 = synth.normal_bf16(12802, (1, K3))
    xin = dev_bf16(x0, device)

    def chain(step):
        x = xin
        for l in range(L):
            x = mods[l].forward(x, ids=ids_d[l][step:step + 1], weights=w_d[l][step:step + 1])
        return x

    announce(f"graph-captured chained decode: {L} layers, ids path, K={K3}")
    out = chain(0)
    eager = host_bits(out).copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured_out = chain(0)
    assert captured_out.data_ptr() == out.data_ptr()
    for rep in range(3):
        out.zero_()
        g.replay()
        assert np.array_equal(host_bits(out), eager), f"replay {rep} differs from the eager chain"
        # eager work between replays: the other routing step on another input
        xin.copy_(dev_bf16(x1, device))
        chain(1)
        torch.cuda.synchronize()
        xin.copy_(dev_bf16(x0, device))
    x_ref = x0
    for l in range(L):
        ids, wt = routing[l][0][:1], routing[l][1][:1]
        x_ref = mx.moe_layer(x_ref, _host_expert_fn(layers[l]), ids, wt, O3)
    assert_close(eager, x_ref, "graph-captured three-layer chain vs the oracle's chain")
    del g, mods, layers
    torch.cuda.empty_cache()


# ------------------------------------------- the reference engine's router --

@pytest.mark.parametrize("T,E,K", [(1, 256, 4096), (5, 200, 1000), (16, 256, 4096)])
def test_router_logits(device, T, E, K):
    announce(f"mxfp4_moe_router_logits T={T} E={E} K={K}")
    x = synth.normal_bf16(13000 + T, (T, K))
    wg = synth.normal_bf16(13010 + E, (E, K), 0.0, 0.02)
    got = gb.router_logits(dev_bf16(x, device), dev_bf16(wg, device)).cpu().numpy()
    ref = mx.router_logits(x, wg)
    bound = (np.abs(mx.bf16_to_f32(x)).astype(np.float64) @ np.abs(mx.bf16_to_f32(wg)).astype(np.float64).T) * 2e-6
    assert np.all(np.abs(got.astype(np.float64) - ref) <= bound + 1e-30)


def _softplus_edge_logits():
    rng = np.random.default_rng(13100)
    cases = [("random", (rng.standard_normal((8, 256)) * 2).astype(np.float32), 6)]
    cases.append(("halves", (np.round(rng.standard_normal((4, 256)) * 2) / 2).astype(np.float32), 6))
    z = np.zeros((2, 256), dtype=np.float32)
    z[:, ::3] = -0.0
    z[0, [7, 90, 200]] = [1.0, 2.0, 1.0]
    cases.append(("signed zeros", z, 6))
    ni = np.full((2, 256), -np.inf, dtype=np.float32)
    ni[0, [3, 77, 130]] = [0.5, -2.0, 0.5]
    ni[1, [5, 6]] = [np.inf, 1.0]
    cases.append(("infinities", ni, 6))
    na = rng.standard_normal((2, 256)).astype(np.float32)
    na[:, 1::4] = np.nan
    cases.append(("nan entries", na, 6))
    cases.append(("very negative", (rng.standard_normal((2, 256)) - 60).astype(np.float32), 6))
    cases.append(("E=300 k=8", rng.standard_normal((3, 300)).astype(np.float32), 8))
    cases.append(("E=1024 k=16", (np.round(rng.standard_normal((2, 1024)) * 4) / 4).astype(np.float32), 16))
    return cases


@pytest.mark.parametrize("name,logits,k", _softplus_edge_logits(), ids=lambda v: v if isinstance(v, str) else "")
def test_route_topk_sqrt_softplus(device, name, logits, k):
    """Ids bit-exact with the oracle (ties to the lower index, NaN never
    before a number); weights within float rounding of the score functions."""
    announce(f"mxfp4_moe_route_topk score_mode=1 {name} E={logits.shape[1]} k={k}")
    ids, w = gb.route_topk(dev_f32(logits, device), k, gb.SCORE_SQRT_SOFTPLUS, 1.5)
    rids, rw = mx.route_sqrt_softplus_topk(logits, k, 1.5)
    assert np.array_equal(ids.cpu().numpy(), rids), name
    assert np.allclose(w.cpu().numpy(), rw, rtol=2e-6, atol=1e-12, equal_nan=True), name


@pytest.mark.parametrize("name,logits,k", _softplus_edge_logits()[:5], ids=lambda v: v if isinstance(v, str) else "")
def test_moe_layer_gated_sqrt_softplus_one_token(device, name, logits, k):
    """The one-token dispatch ranks the scores inside stage A; its published
    ids and weights equal the routing kernel's for the same logits (here fed
    through mxfp4_moe_routed_dispatch's scoring by a one-hot router)."""
    E = logits.shape[1]
    K, H, O = 2048, 64, 128
    announce(f"routed dispatch one-token scoring {name} E={E} k={k}")
    w = moe.make_moe_weights(13200 + E, E, K, H, O, device)
    # x = e_0 and W_gate[:, 0] = bf16(logits): the router GEMV returns the logits
    # themselves when they are bf16 values (the rows here are rounded to bf16).
    for t in range(logits.shape[0]):
        row = mx.bf16_to_f32(mx.bf16_round(logits[t]))
        x = np.zeros((1, K), np.uint16)
        x[0, 0] = 0x3F80
        wg = np.zeros((E, K), np.uint16)
        wg[:, 0] = mx.bf16_round(row)
        ids_out = torch.empty(1, k, dtype=torch.int32, device=device)
        w_out = torch.empty(1, k, dtype=torch.float32, device=device)
        gb.mxfp4_moe_routed_dispatch(dev_bf16(x, device), dev_bf16(wg, device), w.W1, w.W3, w.W2, k, 1.5,
                                     ids_out=ids_out, weights_out=w_out)
        rids, rw = mx.route_sqrt_softplus_topk(row[None, :], k, 1.5)
        assert np.array_equal(ids_out.cpu().numpy(), rids), f"{name} row {t}"
        assert np.allclose(w_out.cpu().numpy(), rw, rtol=2e-6, atol=1e-12, equal_nan=True), f"{name} row {t}"
    del w
    torch.cuda.empty_cache()


def _multi_token_gating_cases():
    """Logit sets for the layer's gating of several tokens:
    shared and identical tokens (many pairs per slot), ties, signed zeros,
    -inf (with a row of all -inf), NaN, the most entries (T = 16, top-16 of
    1024 experts) and every expert routed (E = 8)."""
    rng = np.random.default_rng(13500)
    cases = []
    sh = rng.standard_normal((16, 256)).astype(np.float32)
    sh[::2, 3] += 8.0
    sh[::2, 200] += 8.0
    cases.append(("shared experts", sh, 8))
    cases.append(("identical tokens", np.tile(rng.standard_normal((1, 256)), (16, 1)), 8))
    cases.append(("halves", np.round(rng.standard_normal((5, 256)) * 2) / 2, 8))
    z = np.zeros((4, 256), dtype=np.float32)
    z[:, ::3] = -0.0
    z[0, [7, 90, 200]] = [1.0, 2.0, 1.0]
    z[1, 250] = -1.0
    z[2] = np.round(rng.standard_normal(256))
    cases.append(("signed zeros", z, 8))
    ni = np.full((3, 256), -np.inf, dtype=np.float32)
    ni[0, [3, 77, 130]] = [0.5, -2.0, 0.5]
    ni[2] = rng.standard_normal(256)
    cases.append(("minus inf", ni, 8))
    na = rng.standard_normal((3, 256)).astype(np.float32)
    na[:, 1::4] = np.nan
    cases.append(("nan entries", na, 8))
    cases.append(("E=1024 k=16 T=16", np.round(rng.standard_normal((16, 1024)) * 4) / 4, 16))
    cases.append(("E=200 k=16 T=9", rng.standard_normal((9, 200)), 16))
    cases.append(("E=300 k=5 T=7", rng.standard_normal((7, 300)), 5))
    cases.append(("E=8 k=8 T=2", rng.standard_normal((2, 8)), 8))
    return cases


@pytest.mark.parametrize("name,logits,k", _multi_token_gating_cases(),
                         ids=lambda v: v if isinstance(v, str) else "")
def test_moe_layer_multi_token_gating(device, name, logits, k):
    """The layer of 2 to 16 tokens gates on the device (the routing kernel
    ranks the logits, then stage A and stage B): the ids equal the oracle's,
    the weights agree to float rounding, the output matches the oracle on
    those ids, and its bits equal those of the grouped GEMV given the
    published ids and weights (the routing kernel's ids path)."""
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    K, H, O = 2048, (32 if E > 256 else 64), 128
    announce(f"mxfp4_moe_layer gating in stage A: {name} T={T} E={E} k={k} K={K} H={H} O={O}")
    w = moe.make_moe_weights(13600 + E, E, K, H, O, device)
    x = synth.normal_bf16(13700 + T, (T, K))
    xd = dev_bf16(x, device)
    ids_out = torch.empty(T, k, dtype=torch.int32, device=device)
    w_out = torch.empty(T, k, dtype=torch.float32, device=device)
    out = host_bits(gb.mxfp4_moe_layer(xd, dev_f32(logits, device), w.W1, w.W3, w.W2, k,
                                       ids_out=ids_out, weights_out=w_out))
    rids, rw = mx.route_sigmoid_topk(logits, k)
    assert np.array_equal(ids_out.cpu().numpy(), rids), name
    # a row whose logits are all -inf gets 0/0 weights in both
    assert np.allclose(w_out.cpu().numpy(), rw, rtol=1e-5, atol=1e-6, equal_nan=True), name
    routed = host_bits(gb.mxfp4_moe_grouped_gemv(xd, w.W1, w.W3, w.W2, ids_out, w_out))
    assert np.array_equal(out, routed), f"{name}: gated layer differs from the routing kernel's path"
    rows = np.all(np.isfinite(rw), axis=1)
    ref = mx.moe_layer(x[rows], _host_expert_fn(w), rids[rows], rw[rows], O, n_experts=E)
    assert_close(out[rows], ref, name)
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("T", [1, 4])
def test_routed_dispatch_config_shapes(device, cfg3_layer, T):
    """The reference engine's routed dispatch at its shapes (256 experts,
    hidden 4096, expert ff 2048, top-6, routed scale 1.5) on the device:
    the router GEMV's logits route exactly as the oracle routes the same
    logits, and the output matches the oracle's layer on those ids."""
    w = cfg3_layer
    k = 6
    announce(f"mxfp4_moe_routed_dispatch T={T} E={E3} K={K3} top-{k}")
    x = synth.normal_bf16(13300 + T, (T, K3))
    wg = synth.normal_bf16(13310, (E3, K3), 0.0, 0.02)
    xd, wgd = dev_bf16(x, device), dev_bf16(wg, device)
    ids_out = torch.empty(T, k, dtype=torch.int32, device=device)
    w_out = torch.empty(T, k, dtype=torch.float32, device=device)
    out = host_bits(gb.mxfp4_moe_routed_dispatch(xd, wgd, w.W1, w.W3, w.W2, k, 1.5,
                                                 ids_out=ids_out, weights_out=w_out))
    logits = gb.router_logits(xd, wgd).cpu().numpy()
    assert np.allclose(logits, mx.router_logits(x, wg), rtol=0, atol=1e-4)
    rids, rw = mx.route_sqrt_softplus_topk(logits, k, 1.5)
    ids = ids_out.cpu().numpy()
    assert np.array_equal(ids, rids)
    assert np.allclose(w_out.cpu().numpy(), rw, rtol=2e-6)
    ref = mx.moe_layer(x, _host_expert_fn(w), rids, rw, O3)
    assert_close(out, ref, f"routed dispatch T={T}")
    # bit-deterministic across calls
    again = host_bits(gb.mxfp4_moe_routed_dispatch(xd, wgd, w.W1, w.W3, w.W2, k, 1.5))
    assert np.array_equal(again, out)


@pytest.mark.parametrize("T", [1, 4])
def test_gate_swiglu_then_down_equals_layer(device, cfg3_layer, T):
    """mxfp4_moe_gate_swiglu followed by mxfp4_moe_down (the bench's per-launch
    timing split) gives the bits of mxfp4_moe_layer, with the same routing."""
    w = cfg3_layer
    announce(f"mxfp4_moe_gate_swiglu + mxfp4_moe_down T={T}")
    x = dev_bf16(synth.normal_bf16(13400 + T, (T, K3)), device)
    logits = dev_f32(synth.gating_logits(13410 + T, T, E3), device)
    ids_a = torch.empty(T, 8, dtype=torch.int32, device=device)
    w_a = torch.empty(T, 8, dtype=torch.float32, device=device)
    st = gb.MoEStages(w.W1, w.W3, w.W2, T, 8, device)
    st.gate_swiglu(x, logits, ids_a, w_a)
    split = host_bits(st.down(torch.empty(T, O3, dtype=torch.bfloat16, device=device)))
    ids_b = torch.empty(T, 8, dtype=torch.int32, device=device)
    w_b = torch.empty(T, 8, dtype=torch.float32, device=device)
    whole = host_bits(gb.mxfp4_moe_layer(x, logits, w.W1, w.W3, w.W2, 8, ids_out=ids_b, weights_out=w_b))
    assert np.array_equal(split, whole)
    assert np.array_equal(ids_a.cpu().numpy(), ids_b.cpu().numpy())
    assert np.array_equal(w_a.cpu().numpy(), w_b.cpu().numpy())
