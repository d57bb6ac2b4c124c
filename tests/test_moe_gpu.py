"""GPU parity of the routed-MoE layer against the oracle, through the C ABI.

Routing: the ordered top-k must equal the oracle's for every token whose
top-(k+1) reference logits are separated by more than twice the router's
fp32 error bound (K * 2^-24 * sum|w x|); the set must match wherever the
k-th / (k+1)-th gap alone clears that bound.
Outputs: per element, |y_gpu - y_oracle| <= 1e-4 * S_i where S_i is the
absolute-value sum of the final contraction,
  S_i = sum_r |w_r| sum_f |Wd_r[i,f] h_r[f]| + |s| sum_f |Wsd[i,f] hs[f]|,
evaluated in float64 from the oracle's exact dequantised weights.
"""
import dataclasses
import os

import numpy as np
import pytest

import oracle
from llambda_amd import ggml, synthetic
from llambda_amd.hip_backend import HipBackendError
from llambda_amd.moe import (NEMOTRON_H, QWEN3NEXT, HipMoeSession, MoeLayerInputError,
                             select_top_k, synthetic_nemotron_h, synthetic_qwen3next)

from helpers import REL

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)


def _dq(pair, rows, columns, first_row=0):
    t, data = pair
    rb = ggml.row_bytes(t, columns)
    chunk = data[first_row * rb:(first_row + rows) * rb]
    return oracle.dequantize(t, chunk, rows * columns).reshape(rows, columns).astype(np.float64)


def _silu(v):
    return v / (1.0 + np.exp(-v))


def layer64(layer, x, idx, w, shared_w):
    """The layer's output under the routing (idx, w) and the shared weights,
    and S_i per token (see module docstring), both in float64 from the
    exact dequantised weights (a layer without latent projections)."""
    H, F, Fs = layer.hidden, layer.expert_ffn, layer.shared_ffn
    Y = np.zeros((x.shape[0], H))
    S = np.zeros((x.shape[0], H))
    x64 = x.astype(np.float64)
    by_expert = {}
    for t in range(x.shape[0]):
        for r in range(layer.top_k):
            by_expert.setdefault(int(idx[t, r]), []).append((t, r))
    for e, pairs in by_expert.items():
        ts = np.array([p[0] for p in pairs])
        ws = np.array([w[p] for p in pairs], dtype=np.float64)
        up = _dq(layer.up, F, H, e * F) @ x64[ts].T
        if layer.variant == QWEN3NEXT:
            g = _dq(layer.gate, F, H, e * F) @ x64[ts].T
            h = _silu(g) * up
        else:
            h = np.maximum(up, 0.0) ** 2
        down = _dq(layer.down, H, F, e * H)
        # a token may take an expert once: np.add.at for the general case
        np.add.at(Y, ts, ws[:, None] * (down @ h).T)
        np.add.at(S, ts, np.abs(ws)[:, None] * (np.abs(down) @ np.abs(h)).T)
    if Fs:
        up = _dq(layer.shared_up, Fs, H) @ x64.T
        if layer.variant == QWEN3NEXT:
            h = _silu(_dq(layer.shared_gate, Fs, H) @ x64.T) * up
        else:
            h = np.maximum(up, 0.0) ** 2
        down = _dq(layer.shared_down, H, Fs)
        Y += shared_w[:, None] * (down @ h).T
        S += np.abs(shared_w)[:, None] * (np.abs(down) @ np.abs(h)).T
    return Y, S


def output_bounds(layer, x, idx, w, shared_w):
    """S_i per token (see module docstring), float64."""
    return layer64(layer, x, idx, w, shared_w)[1]


def _shared_weights(layer, x):
    if layer.variant == QWEN3NEXT and layer.shared_ffn:
        return np.array([oracle.sigmoid(float(oracle.dot_product(layer.shared_gate_inp, xt)))
                         for xt in x], dtype=np.float64)
    return np.ones(x.shape[0])


def router_bound(layer, x):
    """K * 2^-24 * sum_i |w_i x_i| per token: a bound on the serial fp32 router
    sum's deviation from the exact dot (plus the GPU's own, same order)."""
    a = np.abs(layer.router.astype(np.float64)) @ np.abs(x.astype(np.float64)).T
    return (layer.hidden * 2.0 ** -24) * a.max(axis=0)


def check_layer(layer, x, label):
    print(f"moe {label} tokens={x.shape[0]}", flush=True)
    session = HipMoeSession(layer)
    try:
        y, idx, w, logits = session.run(x, with_routing=True)
    finally:
        session.close()
    ref = oracle.moe_forward(layer, x, threads=THREADS)
    k = layer.top_k
    # routing
    rb = router_bound(layer, x)
    margins = []
    for t in range(x.shape[0]):
        row = ref.router_logits[t]
        order = np.argsort(-row, kind="stable")[:k + 1]
        top = row[order]
        gap_k = top[k - 1] - top[k] if k < row.size else np.inf
        if gap_k > 2 * rb[t]:
            assert set(idx[t]) == set(ref.top_indices[t]), f"{label} token {t}: expert set differs"
        if np.all(-np.diff(top) > 2 * rb[t]):
            assert np.array_equal(idx[t], ref.top_indices[t]), f"{label} token {t}: order differs"
        margins.append(gap_k / max(rb[t], 1e-30))
    # outputs, against the oracle's routing, for every token whose expert
    # set matches (an order that differs only moves the rank-order sums'
    # rounding, which the bound covers)
    S = output_bounds(layer, x, ref.top_indices, ref.top_weights, _shared_weights(layer, x))
    same_set = np.array([set(idx[t]) == set(ref.top_indices[t]) for t in range(x.shape[0])])
    same = np.array([np.array_equal(idx[t], ref.top_indices[t]) for t in range(x.shape[0])])
    err = np.abs(y.astype(np.float64) - ref.y.astype(np.float64))
    bad = (err > REL * S) & same_set[:, None]
    assert not bad.any(), (f"{label}: {int(bad.sum())} outputs exceed 1e-4*S "
                           f"(max ratio {np.max(err[same_set] / np.maximum(S[same_set], 1e-300)):.3e})")
    assert same_set.mean() > 0.9, f"{label}: expert sets matched on only {same_set.mean():.2%} of tokens"
    # gating weights of identically routed tokens agree up to the router
    # logits' rounding (|d sigmoid / dl| <= 1/4 and the renormalisation keeps
    # the scale): |dw| <= 1e-6 |w| + router bound; a token whose set matches
    # in another order carries the same weights per expert
    dw = np.abs(w.astype(np.float64) - ref.top_weights)
    ok = dw <= 1e-6 * np.abs(ref.top_weights) + rb[:, None]
    assert np.all(ok[same]), f"{label}: gating weights differ beyond the router bound"
    for t in np.nonzero(same_set & ~same)[0]:
        got_w = dict(zip(idx[t].tolist(), w[t].astype(np.float64)))
        for e, rw in zip(ref.top_indices[t].tolist(), ref.top_weights[t]):
            assert abs(got_w[e] - rw) <= 1e-6 * abs(rw) + 2 * rb[t], f"{label} token {t}"
    print(f"{label}: {int(same_set.sum())} of {x.shape[0]} tokens checked "
          f"({int((same_set & ~same).sum())} in another rank order)", flush=True)
    return y, idx


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_qwen3next_decode(hip, seed):
    rng = np.random.default_rng(seed)
    layer = synthetic_qwen3next(rng)
    x = synthetic.activations(rng, 1, layer.hidden)
    check_layer(layer, x, f"qwen3next seed={seed}")


def test_qwen3next_prefill_256(hip):
    rng = np.random.default_rng(100)
    layer = synthetic_qwen3next(rng)
    x = synthetic.activations(rng, 256, layer.hidden)
    y, idx = check_layer(layer, x, "qwen3next prefill")
    # a token run alone (the single-token pipeline: K split over four
    # wavefronts) routes exactly as inside the batch (the router's order is
    # the same for every batch size) and agrees within the parity bound
    sub = list(range(0, 256, 37))
    ref = oracle.moe_forward(layer, x[sub], threads=THREADS)
    S = output_bounds(layer, x[sub], ref.top_indices, ref.top_weights,
                      _shared_weights(layer, x[sub]))
    session = HipMoeSession(layer)
    try:
        for j, t in enumerate(sub):
            y1, i1, _, _ = session.run(x[t:t + 1], with_routing=True)
            np.testing.assert_array_equal(i1[0], idx[t])
            err = np.abs(y1[0].astype(np.float64) - y[t].astype(np.float64))
            assert np.all(err <= 2 * REL * S[j]), f"token {t}: single run differs from the batch"
    finally:
        session.close()


def test_nemotron_h_decode_and_batch(hip):
    rng = np.random.default_rng(7)
    layer = synthetic_nemotron_h(rng)
    x = synthetic.activations(rng, 48, layer.hidden)
    check_layer(layer, x, "nemotron")
    y1, _ = check_layer(layer, x[:1], "nemotron decode")


def test_nemotron_h_1024_batch_invariance(hip):
    rng = np.random.default_rng(8)
    layer = synthetic_nemotron_h(rng)
    x = synthetic.activations(rng, 1024, layer.hidden)
    session = HipMoeSession(layer)
    try:
        y, idx, w, logits = session.run(x, with_routing=True)
        assert np.isfinite(y).all()
        # expert load is skewed by the Zipf bias
        counts = np.bincount(idx.reshape(-1), minlength=layer.expert_count)
        assert counts.max() > 4 * counts.mean()
        for t0 in (0, 511, 1000):
            yc = session.run(x[t0:t0 + 24])
            np.testing.assert_array_equal(yc, y[t0:t0 + 24])
    finally:
        session.close()
    # every 16th token of the full batch against the oracle, token by token
    # (the reference has no batched path), under the same routing and output
    # rules as check_layer
    sub = np.arange(0, 1024, 16)
    print(f"nemotron B=1024: oracle on {sub.size} tokens", flush=True)
    ref = oracle.moe_forward(layer, x[sub], threads=THREADS)
    rb = router_bound(layer, x[sub])
    k = layer.top_k
    same_set = np.zeros(sub.size, dtype=bool)
    for j, t in enumerate(sub):
        row = ref.router_logits[j]
        top = row[np.argsort(-row, kind="stable")[:k + 1]]
        if top[k - 1] - top[k] > 2 * rb[j]:
            assert set(idx[t]) == set(ref.top_indices[j]), f"token {t}: expert set differs"
        if np.all(-np.diff(top) > 2 * rb[j]):
            assert np.array_equal(idx[t], ref.top_indices[j]), f"token {t}: order differs"
        same_set[j] = set(idx[t]) == set(ref.top_indices[j])
    assert same_set.mean() > 0.9
    S = output_bounds(layer, x[sub], ref.top_indices, ref.top_weights,
                      _shared_weights(layer, x[sub]))
    err = np.abs(y[sub].astype(np.float64) - ref.y.astype(np.float64))
    bad = (err > REL * S) & same_set[:, None]
    assert not bad.any(), f"B=1024: {int(bad.sum())} outputs of the sampled tokens exceed 1e-4*S"
    # every token of the batch against the float64 restatement of the
    # expert products and the combine under the device's own routing (its
    # expert set and gating weights, checked above on the sampled tokens):
    # the per-chunk arithmetic of every hot expert's every 64-pair chunk
    print("nemotron B=1024: float64 products of all 1024 tokens", flush=True)
    Y64, S64 = layer64(layer, x, idx, w.astype(np.float64), np.ones(x.shape[0]))
    err = np.abs(y.astype(np.float64) - Y64)
    bad = err > REL * S64
    assert not bad.any(), (f"B=1024: {int(bad.sum())} outputs exceed 1e-4*S against float64 "
                           f"(tokens {sorted(set(np.nonzero(bad)[0].tolist()))[:10]})")


# One token through each single-token launch sequence: the up launch that
# selects and gates the token itself and the down launch that combines
# (no shared expert; K not a multiple of 256; top-k of 1 and of 12 over 600
# experts, 16 logits per lane), and the sequence with a separate top-k
# launch and combine (a shared expert of another weight type).
def _single_token_layer(case, rng):
    if case == "qwen no shared":
        return synthetic_qwen3next(rng, hidden=512, experts=32, top_k=4, ffn=256, shared_ffn=0)
    if case == "nemotron no shared, partial K":
        return synthetic_nemotron_h(rng, hidden=512, experts=32, top_k=4, ffn=96, shared_ffn=0,
                                    expert_type=ggml.Q5_0, down_type=ggml.Q5_0)
    if case == "nemotron shared, partial K":
        return synthetic_nemotron_h(rng, hidden=512, experts=32, top_k=3, ffn=224,
                                    shared_ffn=160, expert_type=ggml.Q8_0, down_type=ggml.Q8_0)
    if case == "qwen top-1":
        return synthetic_qwen3next(rng, hidden=512, experts=16, top_k=1, ffn=256, shared_ffn=256)
    if case == "qwen top-12 of 600":
        return synthetic_qwen3next(rng, hidden=256, experts=600, top_k=12, ffn=64, shared_ffn=64,
                                   gate_type=ggml.Q8_0, down_type=ggml.Q8_0)
    assert case == "qwen shared of another type"
    layer = synthetic_qwen3next(rng, hidden=512, experts=32, top_k=4, ffn=256, shared_ffn=256)
    gen = synthetic.packed
    return dataclasses.replace(
        layer, shared_gate=(ggml.Q8_0, gen(ggml.Q8_0, rng, 256, 512)),
        shared_up=(ggml.Q8_0, gen(ggml.Q8_0, rng, 256, 512)),
        shared_down=(ggml.Q5_0, gen(ggml.Q5_0, rng, 512, 256)))


@pytest.mark.parametrize("case", ["qwen no shared", "nemotron no shared, partial K",
                                  "nemotron shared, partial K", "qwen top-1",
                                  "qwen top-12 of 600", "qwen shared of another type"])
def test_single_token_sequences(hip, case):
    rng = np.random.default_rng(sum(map(ord, case)))
    layer = _single_token_layer(case, rng)
    for t in range(3):
        check_layer(layer, synthetic.activations(rng, 1, layer.hidden), f"{case} token {t}")


def test_small_qwen_shapes(hip):
    rng = np.random.default_rng(9)
    layer = synthetic_qwen3next(rng, hidden=256, experts=20, top_k=3, ffn=64, shared_ffn=32,
                                gate_type=ggml.Q8_0, down_type=ggml.Q5_0)
    x = synthetic.activations(rng, 13, layer.hidden)
    check_layer(layer, x, "qwen small")


def test_double_pipeline_shared_activations_ragged(hip):
    """Batches of at most 16 pairs per expert on 32-weight blocks: the
    gate|up products (Q5_0, 16-byte fragments) share the chunk's activations
    through LDS, the down products (Q8_0) run the one-stage loop.  ffn 224:
    the gate|up rows end inside a workgroup (two of its waves have none) and
    the down K ends inside a chunk.  Against the oracle, and bit for bit
    against a batch of 5."""
    rng = np.random.default_rng(44)
    layer = synthetic_qwen3next(rng, hidden=512, experts=16, top_k=4, ffn=224, shared_ffn=224,
                                gate_type=ggml.Q5_0, down_type=ggml.Q8_0)
    x = synthetic.activations(rng, 24, layer.hidden)
    assert 24 * layer.top_k / layer.expert_count <= 16
    y, _ = check_layer(layer, x, "double pipeline, shared activations")
    session = HipMoeSession(layer)
    try:
        np.testing.assert_array_equal(session.run(x[3:8]), y[3:8])
    finally:
        session.close()


def test_router_expert_groups_ragged(hip):
    """300 tokens (19 token tiles, the last partial) take the router launch
    with eight expert tiles per workgroup; 40 experts + the shared gate row
    are 41 router rows, three tiles of one group, the last partial.  Against
    the oracle, and bit for bit against the same tokens in a batch of 20 (one
    expert tile per workgroup)."""
    rng = np.random.default_rng(42)
    layer = synthetic_qwen3next(rng, hidden=768, experts=40, top_k=4, ffn=64, shared_ffn=64,
                                gate_type=ggml.Q8_0, down_type=ggml.Q5_0)
    x = synthetic.activations(rng, 300, layer.hidden)
    y, _ = check_layer(layer, x, "router expert groups")
    session = HipMoeSession(layer)
    try:
        np.testing.assert_array_equal(session.run(x[280:300]), y[280:300])
    finally:
        session.close()


# Batches whose average load per expert (tokens * k / E) is above 16 pairs:
# chunks of two token tiles (the wide pipeline) against the oracle.  Every
# weight type, relu^2 (one matrix) and silu-gate (two side by side) products.
@pytest.mark.parametrize("variant,types,tokens", [
    ("nemotron", (ggml.Q5_0, ggml.Q5_0), 64), ("nemotron", (ggml.Q5_0, ggml.Q5_0), 96),
    ("nemotron", (ggml.Q4_K, ggml.Q6_K), 96), ("nemotron", (ggml.Q8_0, ggml.Q8_0), 96),
    ("qwen", (ggml.Q4_K, ggml.Q6_K), 64), ("qwen", (ggml.Q4_K, ggml.Q6_K), 96),
    ("qwen", (ggml.Q8_0, ggml.Q5_0), 96)])
def test_long_chunks(hip, variant, types, tokens):
    rng = np.random.default_rng(12 + tokens)
    if variant == "nemotron":
        layer = synthetic_nemotron_h(rng, hidden=512, experts=8, top_k=3, ffn=256, shared_ffn=256,
                                     expert_type=types[0], down_type=types[1])
    else:
        layer = synthetic_qwen3next(rng, hidden=512, experts=8, top_k=3, ffn=256, shared_ffn=256,
                                    gate_type=types[0], down_type=types[1])
    avg = tokens * layer.top_k / layer.expert_count
    assert 16 < avg
    x = synthetic.activations(rng, tokens, layer.hidden)
    y, _ = check_layer(layer, x, f"{variant} {types} long chunks")
    # the same tokens in a batch of 5 (one-tile chunks) give the same bits
    session = HipMoeSession(layer)
    try:
        np.testing.assert_array_equal(session.run(x[3:8]), y[3:8])
    finally:
        session.close()


# The group pipeline (every tensor a 32-weight type, 64-pair chunks) where
# rows end inside a wave and whole waves lie past the last row: ffn 160 (up
# rows 128-159 in a wave of 64, the fourth wave past them), hidden 544 (down
# rows 512-543, then three waves past them), a shared expert of 96 rows.
@pytest.mark.parametrize("types", [(ggml.Q5_0, ggml.Q5_0), (ggml.Q8_0, ggml.Q8_0)])
def test_group_pipeline_ragged_rows(hip, types):
    rng = np.random.default_rng(41)
    layer = synthetic_nemotron_h(rng, hidden=544, experts=8, top_k=3, ffn=160, shared_ffn=96,
                                 expert_type=types[0], down_type=types[1])
    tokens = 72
    assert tokens * layer.top_k / layer.expert_count > 16
    x = synthetic.activations(rng, tokens, layer.hidden)
    y, _ = check_layer(layer, x, f"{types} ragged group pipeline")
    session = HipMoeSession(layer)
    try:
        np.testing.assert_array_equal(session.run(x[3:8]), y[3:8])
    finally:
        session.close()


# The group pipeline with the shared expert in another 32-weight type than
# the routed ones (Q8_0 beside Q5_0): routed and shared chunks then take
# separate launches instead of one joint launch.
def test_group_pipeline_separate_shared_launches(hip):
    rng = np.random.default_rng(43)
    layer = synthetic_nemotron_h(rng, hidden=512, experts=8, top_k=3, ffn=256, shared_ffn=160,
                                 expert_type=ggml.Q5_0, down_type=ggml.Q5_0)
    gen = synthetic.packed
    layer = dataclasses.replace(layer, shared_up=(ggml.Q8_0, gen(ggml.Q8_0, rng, 160, 512)),
                                shared_down=(ggml.Q8_0, gen(ggml.Q8_0, rng, 512, 160)))
    tokens = 80
    assert tokens * layer.top_k / layer.expert_count > 16
    x = synthetic.activations(rng, tokens, layer.hidden)
    y, _ = check_layer(layer, x, "group pipeline, separate shared launches")
    session = HipMoeSession(layer)
    try:
        np.testing.assert_array_equal(session.run(x[3:8]), y[3:8])
    finally:
        session.close()


# The same long chunks for 32-weight block experts beside a K-quant shared
# expert: the group pipeline needs every tensor in a 32-weight type, so these
# run on the wide pipeline; ffn 224 makes the down rows 154 (Q5_0) or 238
# (Q8_0) bytes, not dword multiples.  (Layers with Q5_0 rows of an odd
# number of blocks keep 16-pair chunks, whose kernels fit the registers: the
# Q5_0 cases check that path at this batch.)
@pytest.mark.parametrize("variant,types", [
    ("nemotron", (ggml.Q5_0, ggml.Q5_0)), ("nemotron", (ggml.Q8_0, ggml.Q8_0)),
    ("qwen", (ggml.Q8_0, ggml.Q5_0))])
def test_long_chunks_wide_pipeline_32_weight_types(hip, variant, types):
    rng = np.random.default_rng(40)
    gen = synthetic.packed
    if variant == "nemotron":
        layer = synthetic_nemotron_h(rng, hidden=512, experts=8, top_k=3, ffn=224, shared_ffn=256,
                                     expert_type=types[0], down_type=types[1])
        layer = dataclasses.replace(layer, shared_up=(ggml.Q4_K, gen(ggml.Q4_K, rng, 256, 512)),
                                    shared_down=(ggml.Q6_K, gen(ggml.Q6_K, rng, 512, 256)))
    else:
        layer = synthetic_qwen3next(rng, hidden=512, experts=8, top_k=3, ffn=224, shared_ffn=256,
                                    gate_type=types[0], down_type=types[1])
        layer = dataclasses.replace(layer, shared_gate=(ggml.Q4_K, gen(ggml.Q4_K, rng, 256, 512)),
                                    shared_up=(ggml.Q4_K, gen(ggml.Q4_K, rng, 256, 512)),
                                    shared_down=(ggml.Q6_K, gen(ggml.Q6_K, rng, 512, 256)))
    tokens = 96
    assert tokens * layer.top_k / layer.expert_count > 16
    x = synthetic.activations(rng, tokens, layer.hidden)
    check_layer(layer, x, f"{variant} {types} wide pipeline")


def test_nemotron_unnormalised_scaled(hip):
    rng = np.random.default_rng(10)
    layer = synthetic_nemotron_h(rng, hidden=512, experts=64, top_k=4, ffn=256, shared_ffn=0,
                                 expert_type=ggml.Q4_K, down_type=ggml.Q6_K, weights_scale=2.5,
                                 weights_norm=False)
    x = synthetic.activations(rng, 9, layer.hidden)
    check_layer(layer, x, "nemotron no-norm")


def test_nan_input_reports_reference_error(hip):
    rng = np.random.default_rng(11)
    layer = synthetic_qwen3next(rng, hidden=256, experts=16, top_k=2, ffn=64, shared_ffn=64,
                                down_type=ggml.Q8_0)
    x = np.full((1, 256), np.nan, dtype=np.float32)
    session = HipMoeSession(layer)
    try:
        # the reference's own error (status -2), not the backend's condition.
        # Every slot stays (-1, -FLT_MAX), each weight sigmoid(-FLT_MAX) = 0,
        # and the weight-sum check comes before any expert is looked up
        # (llambda.lisp:5364-5375)
        with pytest.raises(MoeLayerInputError,
                           match="Qwen3Next layer router produced non-positive top-k weight sum"
                           ) as info:
            session.run(x)
        assert not isinstance(info.value, HipBackendError)
        # the session stays usable after the error
        good = synthetic.activations(rng, 2, 256)
        assert np.isfinite(session.run(good)).all()
    finally:
        session.close()


def test_nan_input_without_normalisation_reports_the_expert_lookup(hip):
    """Nemotron-H without expert_weights_norm has no weight-sum check: a NaN
    token reaches the expert lookup with index -1 (llambda.lisp:5898-5912)."""
    rng = np.random.default_rng(13)
    layer = synthetic_nemotron_h(rng, hidden=256, experts=16, top_k=2, ffn=64, shared_ffn=0,
                                 expert_type=ggml.Q8_0, down_type=ggml.Q8_0, weights_norm=False)
    session = HipMoeSession(layer)
    try:
        bad = synthetic.activations(rng, 5, 256)
        bad[3] = np.nan
        with pytest.raises(MoeLayerInputError, match="fewer than top-k selectable logits"):
            session.run(bad)
        good = bad[[0, 1, 2, 4]]
        ref = oracle.moe_forward(layer, good)
        y, idx, _, _ = session.run(good, with_routing=True)
        assert np.array_equal(idx, ref.top_indices)
    finally:
        session.close()


def test_non_positive_weight_sum_reports_reference_error(hip):
    """Every biased router logit near -200: each top-k sigmoid rounds to 0 in
    single precision, the normalised Nemotron-H gating finds a zero weight sum
    and the reference signals its error (llambda.lisp:5903-5905)."""
    rng = np.random.default_rng(12)
    layer = synthetic_nemotron_h(rng, hidden=256, experts=16, top_k=2, ffn=64, shared_ffn=64,
                                 expert_type=ggml.Q8_0, down_type=ggml.Q8_0, weights_norm=True)
    layer.router_bias = np.full(16, -200.0, dtype=np.float32)
    layer.layer_index = 7
    x = synthetic.activations(rng, 3, 256)
    with pytest.raises(RuntimeError, match="non-positive top-k weight sum"):
        oracle.moe_forward(layer, x[:1])
    session = HipMoeSession(layer)
    try:
        for batch in (x[:1], x):  # the single-token and the batch pipelines
            with pytest.raises(MoeLayerInputError,
                               match="Nemotron-H MoE layer 7 router produced non-positive "
                                     "top-k weight sum"):
                session.run(batch)
    finally:
        session.close()


def _ref_topk(row, k):
    idx, val = oracle.select_top_k(row, k)
    return idx, val


@pytest.mark.parametrize("n,k", [(512, 10), (128, 6), (1, 1), (1000, 64), (65, 7)])
def test_select_top_k_random(hip, n, k):
    rng = np.random.default_rng(n * 100 + k)
    logits = rng.normal(size=(33, n)).astype(np.float32)
    # ties and specials
    logits[1, :] = 0.0
    logits[2, ::3] = np.nan
    logits[3, : n // 2] = -np.inf
    logits[4, :] = np.float32(-3.4028235e38)
    logits[5, ::2] = -0.0
    logits[6] = np.round(logits[6])
    idx, val = select_top_k(logits, k)
    for t in range(logits.shape[0]):
        ri, rv = _ref_topk(logits[t], k)
        assert np.array_equal(idx[t], ri), t
        assert np.array_equal(val[t].view(np.uint32), rv.view(np.uint32)), t
