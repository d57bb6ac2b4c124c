"""Pin the oracle's MoE layers (llambda.lisp:5321-5426, 5827-5949) against an
independent float64 evaluation built from the dequantised weights, the
closed-form routing (stable descending sort) and the gating formulas.  The
reference's own suite has no test of either MoE function, so these are the
pins.  CPU only."""
import dataclasses

import numpy as np
import pytest

import oracle
from llambda_amd import ggml, synthetic
from llambda_amd.moe import NEMOTRON_H, QWEN3NEXT, synthetic_nemotron_h, synthetic_qwen3next


def dq(pair, rows, columns):
    t, data = pair
    return oracle.dequantize(t, data, rows * columns).reshape(rows, columns).astype(np.float64)


def sig(v):
    return 1.0 / (1.0 + np.exp(-v))


def float64_layer(layer, x):
    H, E, K, F, Fs = (layer.hidden, layer.expert_count, layer.top_k, layer.expert_ffn,
                      layer.shared_ffn)
    up = dq(layer.up, E * F, H).reshape(E, F, H)
    down = dq(layer.down, E * H, F).reshape(E, H, F)
    gate = dq(layer.gate, E * F, H).reshape(E, F, H) if layer.gate else None
    ys, sels, ws = [], [], []
    for xt in x.astype(np.float64):
        logits = layer.router.astype(np.float64) @ xt
        if layer.variant == NEMOTRON_H:
            logits = logits + layer.router_bias
        order = sorted(range(E), key=lambda e: (-logits[e], e))[:K]
        w = sig(logits[order])
        if layer.variant == QWEN3NEXT or layer.expert_weights_norm:
            w = w / w.sum()
        if layer.variant == NEMOTRON_H:
            w = w * layer.expert_weights_scale
        y = np.zeros(H)
        for r, e in enumerate(order):
            u = up[e] @ xt
            if layer.variant == QWEN3NEXT:
                g = gate[e] @ xt
                h = g * sig(g) * u
            else:
                h = np.maximum(u, 0.0) ** 2
            y += w[r] * (down[e] @ h)
        if Fs:
            su = dq(layer.shared_up, Fs, H) @ xt
            if layer.variant == QWEN3NEXT:
                sg = dq(layer.shared_gate, Fs, H) @ xt
                hs = sg * sig(sg) * su
                s = sig(layer.shared_gate_inp.astype(np.float64) @ xt)
            else:
                hs = np.maximum(su, 0.0) ** 2
                s = 1.0
            y += s * (dq(layer.shared_down, H, Fs) @ hs)
        ys.append(y)
        sels.append(order)
        ws.append(w)
    return np.array(ys), np.array(sels), np.array(ws)


def scale_of(y):
    return np.abs(y).max(axis=1, keepdims=True) + 1e-30


@pytest.mark.parametrize("seed", [0, 1])
def test_qwen3next_oracle_vs_float64(seed):
    rng = np.random.default_rng(seed)
    layer = synthetic_qwen3next(rng, hidden=512, experts=24, top_k=4, ffn=256, shared_ffn=256,
                                router_std=0.1)
    x = synthetic.activations(rng, 6, layer.hidden)
    ref = oracle.moe_forward(layer, x, threads=3)
    y64, sel, w64 = float64_layer(layer, x)
    assert np.array_equal(ref.top_indices, sel)
    np.testing.assert_allclose(ref.top_weights, w64, rtol=2e-6)
    assert np.all(np.abs(ref.y - y64) <= 1e-5 * scale_of(y64))


@pytest.mark.parametrize("norm,scale", [(True, 1.0), (False, 2.5)])
def test_nemotron_oracle_vs_float64(norm, scale):
    rng = np.random.default_rng(3)
    layer = synthetic_nemotron_h(rng, hidden=256, experts=16, top_k=3, ffn=96, shared_ffn=64,
                                 router_std=0.1, weights_norm=norm, weights_scale=scale)
    x = synthetic.activations(rng, 5, layer.hidden)
    ref = oracle.moe_forward(layer, x)
    y64, sel, w64 = float64_layer(layer, x)
    assert np.array_equal(ref.top_indices, sel)
    np.testing.assert_allclose(ref.top_weights, w64, rtol=2e-6)
    assert np.all(np.abs(ref.y - y64) <= 1e-5 * scale_of(y64))
    # router logits are reported after the bias (vector-add-bias-in-place)
    np.testing.assert_allclose(ref.router_logits,
                               (x.astype(np.float64) @ layer.router.T.astype(np.float64))
                               + layer.router_bias, rtol=1e-4, atol=1e-5)


def test_qwen3next_nonpositive_sum_is_an_error():
    rng = np.random.default_rng(4)
    layer = synthetic_qwen3next(rng, hidden=256, experts=8, top_k=2, ffn=32, shared_ffn=32,
                                down_type=ggml.Q8_0)
    x = np.full((1, 256), np.nan, dtype=np.float32)
    with pytest.raises(oracle.OracleError, match="Expert index|non-positive"):
        oracle.moe_forward(layer, x)


def test_combine_order_is_rank_order():
    """dest accumulates fl(w * down) in rank order, then the shared term: the
    oracle's output equals that sum formed in float32 from its own pieces."""
    rng = np.random.default_rng(5)
    layer = synthetic_qwen3next(rng, hidden=256, experts=12, top_k=3, ffn=64, shared_ffn=0,
                                down_type=ggml.Q5_0)
    layer.shared_gate_inp = None
    x = synthetic.activations(rng, 1, 256)
    ref = oracle.moe_forward(layer, x)
    H, F = layer.hidden, layer.expert_ffn
    dest = np.zeros(H, dtype=np.float32)
    rb_up = ggml.row_bytes(layer.up[0], H)
    rb_down = ggml.row_bytes(layer.down[0], F)
    for r, e in enumerate(ref.top_indices[0]):
        g = oracle.gemv(layer.gate[0], layer.gate[1][e * F * rb_up:], F, H, x[0])
        u = oracle.gemv(layer.up[0], layer.up[1][e * F * rb_up:], F, H, x[0])
        h = np.array([np.float32(oracle.silu(float(v))) for v in g], dtype=np.float32) * u
        d = oracle.gemv(layer.down[0], layer.down[1][e * H * rb_down:], H, F, h.astype(np.float32))
        dest = (dest + (ref.top_weights[0, r] * d).astype(np.float32)).astype(np.float32)
    assert np.array_equal(dest, ref.y[0])


def float64_latent_layer(layer, x):
    """nemotron-h-moe-ffn-into with its optional ffn_latent_down / ffn_latent_up
    (llambda.lisp:5845-5864, 5883-5887, 5933-5938), each independently, in
    float64 from the dequantised weights."""
    H, E, K, F, Fs = (layer.hidden, layer.expert_count, layer.top_k, layer.expert_ffn,
                      layer.shared_ffn)
    ld = lu = None
    din = dout = H
    if layer.latent_down is not None:
        din = layer.latent_down[1].size // ggml.row_bytes(layer.latent_down[0], H)
        ld = dq(layer.latent_down, din, H)
    if layer.latent_up is not None:
        dout = oracle.columns_of(layer.latent_up[0], layer.latent_up[1].size // H)
        lu = dq(layer.latent_up, H, dout)
    up = dq(layer.up, E * F, din).reshape(E, F, din)
    down = dq(layer.down, E * dout, F).reshape(E, dout, F)
    ys = []
    for xt in x.astype(np.float64):
        logits = layer.router.astype(np.float64) @ xt + layer.router_bias
        order = sorted(range(E), key=lambda e: (-logits[e], e))[:K]
        w = sig(logits[order])
        if layer.expert_weights_norm:
            w = w / w.sum()
        w = w * layer.expert_weights_scale
        ein = ld @ xt if ld is not None else xt
        m = np.zeros(dout)
        for r, e in enumerate(order):
            m += w[r] * (down[e] @ (np.maximum(up[e] @ ein, 0.0) ** 2))
        y = lu @ m if lu is not None else m
        if Fs:
            y += dq(layer.shared_down, H, Fs) @ (np.maximum(dq(layer.shared_up, Fs, H) @ xt, 0.0) ** 2)
        ys.append(y)
    return np.array(ys)


@pytest.mark.parametrize("latent_in,latent_out,latent_type", [
    (128, 128, ggml.Q8_0), (128, 128, ggml.F32), (160, 0, ggml.Q5_0), (0, 96, ggml.Q8_0),
    (96, 160, ggml.Q8_0), (128, 0, ggml.Q6_K), (0, 256, ggml.Q4_K)])
def test_nemotron_latent_oracle_vs_float64(latent_in, latent_out, latent_type):
    rng = np.random.default_rng(11)
    layer = synthetic_nemotron_h(rng, hidden=256, experts=16, top_k=3, ffn=96, shared_ffn=64,
                                 router_std=0.1, expert_type=ggml.Q8_0, down_type=ggml.Q8_0,
                                 latent_in=latent_in, latent_out=latent_out,
                                 latent_type=latent_type)
    x = synthetic.activations(rng, 4, layer.hidden)
    ref = oracle.moe_forward(layer, x, threads=2)
    y64 = float64_latent_layer(layer, x)
    assert np.all(np.abs(ref.y - y64) <= 1e-5 * scale_of(y64))


def _f32(a):
    return (ggml.F32, np.ascontiguousarray(a, dtype=np.float32).view(np.uint8).ravel())


def test_nemotron_latent_permutation_is_exact():
    """ffn_latent_down = I and ffn_latent_up = a permutation P (F32, Lt = H): the
    layer's output is the latent-free layer's output with its entries taken in
    P's order, bit for bit; with ffn_latent_down = I alone it is the latent-free
    output itself, and with ffn_latent_up = P alone the permuted one.  A
    transposed or misplaced latent product fails it."""
    rng = np.random.default_rng(12)
    H = 128
    base = synthetic_nemotron_h(rng, hidden=H, experts=8, top_k=2, ffn=64, shared_ffn=0,
                                router_std=0.1)
    pi = rng.permutation(H)
    assert np.any(pi[pi] != np.arange(H))  # not an involution: P and P^T differ
    perm = np.zeros((H, H), np.float32)
    perm[np.arange(H), pi] = 1.0
    eye = np.eye(H, dtype=np.float32)
    x = synthetic.activations(rng, 3, H)
    want = oracle.moe_forward(base, x).y
    both = dataclasses.replace(base, latent_down=_f32(eye), latent_up=_f32(perm))
    assert np.array_equal(oracle.moe_forward(both, x).y, want[:, pi])
    down_only = dataclasses.replace(base, latent_down=_f32(eye))
    assert np.array_equal(oracle.moe_forward(down_only, x).y, want)
    up_only = dataclasses.replace(base, latent_up=_f32(perm))
    assert np.array_equal(oracle.moe_forward(up_only, x).y, want[:, pi])


def test_latent_projections_only_on_nemotron():
    rng = np.random.default_rng(13)
    layer = synthetic_qwen3next(rng, hidden=256, experts=4, top_k=2, ffn=32, shared_ffn=32,
                                down_type=ggml.Q8_0)
    lat = dataclasses.replace(layer, latent_down=_f32(np.eye(256, dtype=np.float32)))
    with pytest.raises(Exception, match="latent projections belong to Nemotron-H"):
        oracle.moe_forward(lat, synthetic.activations(rng, 1, 256))
