"""The oracle's Llama decode step (oracle_llama_step and its primitives)
pinned against the reference's own known answers (tests.lisp:298-344,
1359-1361), closed forms, and a float64 restatement of the step built from
dequantised weights."""
import math

import numpy as np
import pytest

import oracle
from llambda_amd import ggml
from llambda_amd.llama import LlamaConfig, llama31_rope_factors, synthetic_llama


def test_reference_forward_primitive_kats(kats):
    k = kats["rms_norm"]
    out = oracle.rms_norm(k["x"], k["weight"], k["epsilon"])
    assert np.all(np.abs(out - np.array(k["expect"], dtype=np.float32)) < k["tolerance"])
    k = kats["rope"]
    out = oracle.rope_head(k["x"], k["position"], k["rope_dimension"], k["theta_base"])
    expect = [math.cos(1.0), math.sin(1.0), 5.0, 6.0]
    assert np.all(np.abs(out - np.array(expect, dtype=np.float32)) < k["tolerance"])
    k = kats["softmax"]
    p = oracle.softmax(k["x"])
    assert abs(float(np.sum(p, dtype=np.float64)) - 1.0) < k["tolerance"]
    assert p[0] > p[1] > p[2]


def test_rms_norm_closed_form():
    rng = np.random.default_rng(1)
    x = rng.normal(size=300).astype(np.float32)
    w = rng.uniform(0.5, 1.5, size=300).astype(np.float32)
    out = oracle.rms_norm(x, w, 1e-5).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = x64 * w / np.sqrt(np.mean(x64 * x64) + 1e-5)
    assert np.max(np.abs(out - ref) / np.abs(ref).max()) < 1e-6
    # unit weights: the output's mean square is 1 / (1 + eps / mean(x^2))
    ones = oracle.rms_norm(x, np.ones_like(x), 0.0).astype(np.float64)
    assert abs(np.mean(ones * ones) - 1.0) < 1e-5


@pytest.mark.parametrize("factors", [False, True])
def test_rope_closed_forms(factors):
    rng = np.random.default_rng(2)
    D = 128
    f = llama31_rope_factors(D) if factors else None
    head = rng.normal(size=D).astype(np.float32)
    # position 0 is the identity, bit for bit
    assert np.array_equal(oracle.rope_head(head, 0, D, 500000.0, f), head)
    for pos in (1, 17, 4096):
        out = oracle.rope_head(head, pos, D, 500000.0, f)
        x = head.astype(np.float64).reshape(-1, 2)
        o = out.astype(np.float64).reshape(-1, 2)
        # a rotation keeps each pair's length
        assert np.allclose(np.hypot(o[:, 0], o[:, 1]), np.hypot(x[:, 0], x[:, 1]), rtol=1e-6)
        # the angle of pair i: position / (factor_i * fl32(theta^(2i/D)))
        i = np.arange(D // 2)
        power = np.power(500000.0, 2.0 * i / D).astype(np.float32).astype(np.float64)
        fac = f.astype(np.float64) if f is not None else 1.0
        ang = pos / (fac * power)
        ref0 = x[:, 0] * np.cos(ang) - x[:, 1] * np.sin(ang)
        ref1 = x[:, 0] * np.sin(ang) + x[:, 1] * np.cos(ang)
        tol = 2.0 ** -23 * (np.abs(x[:, 0]) + np.abs(x[:, 1])) + 1e-30
        assert np.all(np.abs(o[:, 0] - ref0) <= tol) and np.all(np.abs(o[:, 1] - ref1) <= tol)


def test_rope_dimension_limits():
    rng = np.random.default_rng(3)
    head = rng.normal(size=16).astype(np.float32)
    # rope_dim 6: pairs 0..2 rotate, the rest is untouched
    out = oracle.rope_head(head, 5, 6, 10000.0)
    assert np.array_equal(out[6:], head[6:]) and not np.array_equal(out[:6], head[:6])
    # 2 factors limit the rotation to 2 pairs; a factor above 1e20 freezes its pair
    out = oracle.rope_head(head, 5, 16, 10000.0, np.array([1.0, 1e21], dtype=np.float32))
    assert np.array_equal(out[2:], head[2:]) and not np.array_equal(out[:2], head[:2])


def test_softmax_against_float64():
    rng = np.random.default_rng(4)
    x = (rng.normal(size=1000) * 5).astype(np.float32)
    p = oracle.softmax(x).astype(np.float64)
    x64 = x.astype(np.float64)
    ref = np.exp(x64 - x64.max())
    ref /= ref.sum()
    assert np.max(np.abs(p - ref) / ref) < 1e-5
    # a single logit is probability 1 exactly
    assert oracle.softmax(np.array([3.5], dtype=np.float32))[0] == 1.0


def attention64(q, kc, vc, n):
    heads, D = q.shape
    kvh = kc.shape[0]
    g = heads // kvh
    out = np.zeros((heads, D))
    for h in range(heads):
        k = kc[h // g, :n].astype(np.float64)
        v = vc[h // g, :n].astype(np.float64)
        s = k @ q[h].astype(np.float64)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[h] = p @ v
    return out


def test_attention_closed_forms():
    rng = np.random.default_rng(5)
    heads, kvh, D, cap = 4, 2, 64, 40
    q = rng.normal(size=(heads, D)).astype(np.float32)
    kc = rng.normal(size=(kvh, cap, D)).astype(np.float32)
    vc = rng.normal(size=(kvh, cap, D)).astype(np.float32)
    # one slot: the value row itself
    out = oracle.attention(q, kc, vc, 1)
    for h in range(heads):
        assert np.array_equal(out[h], vc[h // 2, 0])
    # identical keys: the mean of the value rows
    same = np.repeat(kc[:, :1], cap, axis=1)
    out = oracle.attention(q, same, vc, 30)
    for h in range(heads):
        assert np.allclose(out[h], vc[h // 2, :30].astype(np.float64).mean(axis=0), atol=1e-5)
    # general case against float64; query heads 2h, 2h+1 share kv head h
    out = oracle.attention(q * 0.2, kc, vc, 37)
    ref = attention64(q * 0.2, kc, vc, 37)
    assert np.max(np.abs(out - ref)) < 1e-5 * np.abs(vc).max()


def dequant(t, rows, cols):
    return oracle.dequantize(t[0], t[1], rows * cols).reshape(rows, cols).astype(np.float64)


def llama_step64(w, kv, token, pos):
    """float64 restatement of the step from dequantised weights (kv float64
    [layers][2][kv][cap][D], updated)."""
    c = w.config
    H, D, NH, NKV = c.hidden, c.head_dim, c.head_count, c.kv_head_count
    eps = c.norm_epsilon
    x = dequant((w.token_embd[0], w.token_embd[1][token * ggml.row_bytes(w.token_embd[0], H):]),
                1, H)[0]

    def norm(v, g):
        return v * g / np.sqrt(np.mean(v * v) + eps)

    i = np.arange(D // 2)
    power = np.power(np.float64(c.rope_base), 2.0 * i / D).astype(np.float32).astype(np.float64)
    fac = w.rope_factors.astype(np.float64) if w.rope_factors is not None else 1.0
    ang = pos / (fac * power)
    cs, sn = np.cos(ang), np.sin(ang)

    def rope(v):
        v = v.reshape(-1, D // 2, 2)
        o = np.empty_like(v)
        o[..., 0] = v[..., 0] * cs - v[..., 1] * sn
        o[..., 1] = v[..., 0] * sn + v[..., 1] * cs
        return o.reshape(-1)

    for l, L in enumerate(w.layers):
        xin = norm(x, L.attn_norm.astype(np.float64))
        q = rope(dequant(L.attn_q, NH * D, H) @ xin) / math.sqrt(D)
        k = rope(dequant(L.attn_k, NKV * D, H) @ xin)
        v = dequant(L.attn_v, NKV * D, H) @ xin
        kv[l, 0, :, pos] = k.reshape(NKV, D)
        kv[l, 1, :, pos] = v.reshape(NKV, D)
        ctx = attention64(q.reshape(NH, D), kv[l, 0], kv[l, 1], pos + 1).reshape(-1)
        x = x + dequant(L.attn_output, H, NH * D) @ ctx
        xin = norm(x, L.ffn_norm.astype(np.float64))
        g = dequant(L.ffn_gate, c.ffn, H) @ xin
        u = dequant(L.ffn_up, c.ffn, H) @ xin
        x = x + dequant(L.ffn_down, H, c.ffn) @ (g / (1.0 + np.exp(-g)) * u)
    return dequant(w.output, c.vocab, H) @ norm(x, w.output_norm.astype(np.float64))


TINY = LlamaConfig(hidden=256, layer_count=2, head_count=2, kv_head_count=1, ffn=512, vocab=48,
                   rope_dimension=128, context=16)


@pytest.mark.parametrize("prefill", [0, 9])
def test_llama_step_matches_float64(prefill):
    rng = np.random.default_rng(6 + prefill)
    w = synthetic_llama(rng, TINY)
    c = TINY
    kv = np.zeros((c.layer_count, 2, c.kv_head_count, c.context, c.head_dim), dtype=np.float32)
    kv[:, :, :, :prefill] = rng.normal(size=kv[:, :, :, :prefill].shape)
    kv64 = kv.astype(np.float64)
    for pos, token in ((prefill, 5), (prefill + 1, 31)):
        got = oracle.llama_step(w, kv, token, pos)
        ref = llama_step64(w, kv64, token, pos)
        scale = np.abs(ref).max()
        assert np.max(np.abs(got - ref)) < 2e-5 * scale, (pos, np.max(np.abs(got - ref)) / scale)
        # the cache slot holds the rotated key and the value of this token
        assert np.allclose(kv[:, :, :, pos], kv64[:, :, :, pos], rtol=1e-4,
                           atol=1e-5 * np.abs(kv64[:, :, :, pos]).max())


def test_llama_step_rejects_bad_token_and_position():
    rng = np.random.default_rng(7)
    w = synthetic_llama(rng, TINY)
    kv = np.zeros((2, 2, 1, 16, 128), dtype=np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.llama_step(w, kv, TINY.vocab, 0)
    with pytest.raises(oracle.OracleError):
        oracle.llama_step(w, kv, 0, 16)


# ------------------------------------------------------------------ sampling
def test_reference_sampling_kats(kats):
    k = kats["sampling"]
    tol = k["tolerance"]
    t = k["temperature"]
    assert np.allclose(np.float32(t["x"]) / np.float32(t["t"]), t["expect"], atol=tol)
    r = k["repetition_penalty"]
    assert np.allclose(oracle.repetition_penalty(r["x"], r["history"], r["penalty"]), r["expect"],
                       atol=tol)
    r = k["top_k"]
    assert np.allclose(oracle.top_k(r["x"], r["k"]), r["expect"], atol=tol)
    r = k["top_p"]
    assert np.allclose(oracle.top_p(r["x"], r["p"], r["t"]), r["expect"], atol=tol)
    r = k["probabilities"]
    for roll, want in r["draws"]:
        assert oracle.sample_from_probabilities(r["p"], roll) == want
    for logits, kw, roll, want in k["tokens"]:
        assert oracle.sample_token(logits, random_value=roll, **kw) == want, (logits, kw)
    for logits, kw1, kw2, roll in k["same"]:
        assert oracle.sample_token(logits, random_value=roll, **kw1) == \
            oracle.sample_token(logits, random_value=roll, **kw2)


def test_top_k_is_the_kth_largest_with_ties():
    rng = np.random.default_rng(21)
    for trial in range(30):
        n = int(rng.integers(2, 400))
        x = rng.integers(-20, 20, size=n).astype(np.float32) * np.float32(0.5)  # many ties
        k = int(rng.integers(1, n))
        out = oracle.top_k(x, k)
        cutoff = np.sort(x)[::-1][k - 1]
        assert np.array_equal(out, np.where(x < cutoff, np.float32(-1e30), x))
    x = np.arange(10, dtype=np.float32)
    assert np.array_equal(oracle.top_k(x, 0), x) and np.array_equal(oracle.top_k(x, 10), x)


def test_top_p_against_float64_cumulative():
    rng = np.random.default_rng(22)
    for trial in range(30):
        n = int(rng.integers(2, 300))
        x = (rng.normal(size=n) * 3).astype(np.float32)
        x[rng.random(n) < 0.2] = np.float32(-1e30)
        p = float(rng.uniform(0.05, 0.99))
        T = float(rng.uniform(0.5, 2.0))
        out = oracle.top_p(x, p, T)
        act = np.flatnonzero(x > np.float32(-1e30))
        if act.size <= 1:
            assert np.array_equal(out, x)
            continue
        order = act[np.argsort(-x[act], kind="stable")]
        v = x[order].astype(np.float64) / T
        pr = np.exp(v - v[0])
        pr /= pr.sum()
        cum = np.cumsum(pr)
        j = int(np.argmax(cum >= p)) if (cum >= p).any() else order.size - 1
        # away from rounding ties the cutoff is the value at the first crossing
        if abs(cum[j] - p) > 1e-5 and (j == 0 or abs(cum[j - 1] - p) > 1e-5):
            cutoff = x[order[j]]
            assert np.array_equal(out, np.where(x < cutoff, np.float32(-1e30), x)), trial
