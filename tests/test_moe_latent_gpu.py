"""GPU parity of Nemotron-H MoE layers with ffn_latent_down / ffn_latent_up
(llambda.lisp:5845-5864, 5883-5887, 5933-5938), each present or not, against
the oracle, through the C ABI.

Routing (the router reads x, not the latent vector) follows the margin rule
of test_moe_gpu.  Outputs: per element, |y_gpu - y_oracle| <= 1e-4 * A_i,
where A is the layer evaluated in float64 on absolute values -- |x|, every
dequantised weight's magnitude, |w_r|, relu^2 of the absolute up products --
through ffn_latent_down, the experts, the weighted sum, ffn_latent_up and
the shared expert: the sum of |terms| of every contraction on the way, the
chain's form of the 1e-4 * sum|w x| rule.  Exact cases: with F32
ffn_latent_down = I and ffn_latent_up = a permutation P, the device output
is the latent-free device output (permuted by P) bit for bit.
"""
import dataclasses
import zlib

import numpy as np
import pytest

import oracle
from llambda_amd import ggml, synthetic
from llambda_amd.moe import HipMoeSession, MoeLayerInputError, synthetic_nemotron_h

from helpers import REL
from test_moe_gpu import THREADS, _dq, router_bound

pytestmark = pytest.mark.gpu


def absolute_layer(layer, x, idx, w):
    """A: the layer on absolute values in float64, with the oracle's routing."""
    H, F, Fs = layer.hidden, layer.expert_ffn, layer.shared_ffn
    Li, Lo = layer.latent_in, layer.latent_out
    din, dout = Li or H, Lo or H
    xa = np.abs(x.astype(np.float64))
    ein = xa @ np.abs(_dq(layer.latent_down, Li, H)).T if Li else xa
    m = np.zeros((x.shape[0], dout))
    by_expert = {}
    for t in range(x.shape[0]):
        for r in range(layer.top_k):
            by_expert.setdefault(int(idx[t, r]), []).append((t, r))
    for e, pairs in by_expert.items():
        ts = np.array([p[0] for p in pairs])
        ws = np.abs(np.array([w[p] for p in pairs], dtype=np.float64))
        up = np.abs(_dq(layer.up, F, din, e * F)) @ ein[ts].T
        m[ts] += ws[:, None] * (np.abs(_dq(layer.down, dout, F, e * dout)) @ (up ** 2)).T
    y = m @ np.abs(_dq(layer.latent_up, H, Lo)).T if Lo else m
    if Fs:
        su = np.abs(_dq(layer.shared_up, Fs, H)) @ xa.T
        y = y + (np.abs(_dq(layer.shared_down, H, Fs)) @ (su ** 2)).T
    return y


def check_latent(layer, x, label, session=None):
    print(f"latent {label}: tokens={x.shape[0]} Li={layer.latent_in} Lo={layer.latent_out}",
          flush=True)
    own = session is None
    session = session or HipMoeSession(layer)
    try:
        y, idx, w, _ = session.run(x, with_routing=True)
    finally:
        if own:
            session.close()
    ref = oracle.moe_forward(layer, x, threads=THREADS)
    k = layer.top_k
    rb = router_bound(layer, x)
    for t in range(x.shape[0]):
        row = ref.router_logits[t]
        order = np.argsort(-row, kind="stable")[:k + 1]
        top = row[order]
        gap_k = top[k - 1] - top[k] if k < row.size else np.inf
        if gap_k > 2 * rb[t]:
            assert set(idx[t]) == set(ref.top_indices[t]), f"{label} token {t}: expert set differs"
        if np.all(-np.diff(top) > 2 * rb[t]):
            assert np.array_equal(idx[t], ref.top_indices[t]), f"{label} token {t}: order differs"
    same_set = np.array([set(idx[t]) == set(ref.top_indices[t]) for t in range(x.shape[0])])
    assert same_set.mean() > 0.9, f"{label}: expert sets matched on {same_set.mean():.2%}"
    A = absolute_layer(layer, x, ref.top_indices, ref.top_weights)
    err = np.abs(y.astype(np.float64) - ref.y.astype(np.float64))
    bad = (err > REL * A) & same_set[:, None]
    assert not bad.any(), (f"{label}: {int(bad.sum())} outputs exceed 1e-4*A "
                           f"(max ratio {np.max(err[same_set] / np.maximum(A[same_set], 1e-300)):.3e})")
    print(f"{label}: max err/A {np.max(err[same_set] / np.maximum(A[same_set], 1e-300)):.2e} "
          f"over {int(same_set.sum())} tokens", flush=True)
    return y, idx


# (label, layer keywords, tokens): B=1 with and without a shared expert (the
# latter gates inside the up launch), one-sided layers, and batches that take
# the 16-pair, wide (K-quant experts) and group (32-weight experts, more than
# 16 pairs per expert) pipelines
CASES = [
    ("decode both Q8_0 latents", dict(hidden=512, experts=16, top_k=4, ffn=256, shared_ffn=256,
                                      expert_type=ggml.Q5_0, down_type=ggml.Q5_0, latent_in=256,
                                      latent_out=256, latent_type=ggml.Q8_0), 1),
    ("decode no shared Q5_0 latents", dict(hidden=512, experts=16, top_k=4, ffn=160, shared_ffn=0,
                                           expert_type=ggml.Q8_0, down_type=ggml.Q8_0,
                                           latent_in=192, latent_out=160,
                                           latent_type=ggml.Q5_0), 1),
    ("decode down only", dict(hidden=512, experts=16, top_k=4, ffn=192, shared_ffn=128,
                              expert_type=ggml.Q8_0, down_type=ggml.Q5_0, latent_in=224,
                              latent_type=ggml.Q8_0), 1),
    ("decode up only", dict(hidden=512, experts=16, top_k=4, ffn=192, shared_ffn=128,
                            expert_type=ggml.Q8_0, down_type=ggml.Q8_0, latent_out=288,
                            latent_type=ggml.Q5_0), 1),
    ("batch 40 both", dict(hidden=512, experts=16, top_k=4, ffn=256, shared_ffn=256,
                           expert_type=ggml.Q8_0, down_type=ggml.Q5_0, latent_in=256,
                           latent_out=192, latent_type=ggml.Q8_0), 40),
    ("batch 40 down only", dict(hidden=512, experts=16, top_k=4, ffn=256, shared_ffn=0,
                                expert_type=ggml.Q5_0, down_type=ggml.Q5_0, latent_in=128,
                                latent_type=ggml.Q5_0), 40),
    ("batch 40 up only", dict(hidden=512, experts=16, top_k=4, ffn=256, shared_ffn=320,
                              expert_type=ggml.Q5_0, down_type=ggml.Q8_0, latent_out=352,
                              latent_type=ggml.Q8_0), 40),
    ("group Q5_0 latents", dict(hidden=512, experts=8, top_k=2, ffn=288, shared_ffn=320,
                                expert_type=ggml.Q5_0, down_type=ggml.Q5_0, latent_in=192,
                                latent_out=192, latent_type=ggml.Q5_0), 300),
    ("group Q8_0 latents", dict(hidden=512, experts=8, top_k=2, ffn=288, shared_ffn=320,
                                expert_type=ggml.Q8_0, down_type=ggml.Q5_0, latent_in=256,
                                latent_out=160, latent_type=ggml.Q8_0), 300),
    ("wide K-quant", dict(hidden=512, experts=8, top_k=2, ffn=256, shared_ffn=256,
                          expert_type=ggml.Q4_K, down_type=ggml.Q6_K, latent_in=256,
                          latent_out=256, latent_type=ggml.Q4_K), 120),
]


@pytest.mark.parametrize("label,kw,tokens", CASES, ids=[c[0] for c in CASES])
def test_latent_layer_matches_the_oracle(hip, label, kw, tokens):
    rng = np.random.default_rng(zlib.crc32(label.encode()))
    layer = synthetic_nemotron_h(rng, router_std=0.05, **kw)
    x = synthetic.activations(rng, tokens, layer.hidden)
    check_latent(layer, x, label)


def test_latent_nemotron_shape(hip):
    """Nemotron-H's shape (hidden 2688, 128 experts top-6, ffn 1856, shared
    3712, Q5_0) with 1024-wide latent projections, one token and a batch."""
    rng = np.random.default_rng(21)
    layer = synthetic_nemotron_h(rng, latent_in=1024, latent_out=1024, latent_type=ggml.Q5_0)
    session = HipMoeSession(layer)
    try:
        x = synthetic.activations(rng, 24, layer.hidden)
        check_latent(layer, x[:1], "nemotron shape decode", session)
        check_latent(layer, x, "nemotron shape batch", session)
    finally:
        session.close()


def _f32(a):
    return (ggml.F32, np.ascontiguousarray(a, dtype=np.float32).view(np.uint8).ravel())


@pytest.mark.parametrize("tokens,expert_type", [(2, ggml.Q8_0), (40, ggml.Q5_0),
                                                (300, ggml.Q5_0)])
def test_identity_and_permutation_latents_are_exact(hip, tokens, expert_type):
    """F32 ffn_latent_down = I and ffn_latent_up = P: the experts' input is x
    itself and the output the latent-free output permuted by P, bit for bit,
    in every batch pipeline (a transposed or misplaced latent product, a
    wrong stride or a shared-expert mix-up fails it)."""
    rng = np.random.default_rng(22 + tokens)
    H = 256
    base = synthetic_nemotron_h(rng, hidden=H, experts=8, top_k=2, ffn=128, shared_ffn=0,
                                expert_type=expert_type, down_type=expert_type, router_std=0.1)
    pi = rng.permutation(H)
    assert np.any(pi[pi] != np.arange(H))
    perm = np.zeros((H, H), np.float32)
    perm[np.arange(H), pi] = 1.0
    eye = np.eye(H, dtype=np.float32)
    x = synthetic.activations(rng, tokens, H)
    variants = {
        "both": dataclasses.replace(base, latent_down=_f32(eye), latent_up=_f32(perm)),
        "down": dataclasses.replace(base, latent_down=_f32(eye)),
        "up": dataclasses.replace(base, latent_up=_f32(perm)),
    }
    s0 = HipMoeSession(base)
    try:
        want = s0.run(x)
    finally:
        s0.close()
    for name, layer in variants.items():
        s = HipMoeSession(layer)
        try:
            got = s.run(x)
        finally:
            s.close()
        expect = want if name == "down" else want[:, pi]
        assert np.array_equal(got, expect), f"{name}: {tokens} tokens"


def test_latent_layer_input_error_and_recovery(hip):
    """A NaN token on a latent layer: the reference's error (the final launch,
    after ffn_latent_up, reports the error word), then a good token runs."""
    rng = np.random.default_rng(23)
    layer = synthetic_nemotron_h(rng, hidden=256, experts=16, top_k=2, ffn=64, shared_ffn=64,
                                 expert_type=ggml.Q8_0, down_type=ggml.Q8_0, latent_in=128,
                                 latent_out=128, latent_type=ggml.Q8_0)
    session = HipMoeSession(layer)
    try:
        with pytest.raises(MoeLayerInputError, match="non-positive top-k weight sum"):
            session.run(np.full((1, 256), np.nan, np.float32))
        check_latent(layer, synthetic.activations(rng, 1, 256), "after error", session)
    finally:
        session.close()
