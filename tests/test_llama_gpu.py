"""Parity of the device-resident Llama decode step (llambda_hip_llama_session_*)
with the oracle's step (oracle_llama_step, llambda.lisp:6294-6441).

Bounds: every cache slot the step writes (rotated keys, values) within
1e-4 * sum |w x| of its row, the same bound as a projection, through the
rotation; logits within 1e-3 of the largest |logit| -- the fp32 orders of
the fused GEMV, the chunked attention softmax and the norms differ from the
reference's serial loops, and a wrong head mapping, rotation or cache slot
moves logits by O(1); the full-size token, in addition, every logit within
1e-4 * sum_i |w_ri h_i| of its row (h the oracle's input to the output rows)."""
import dataclasses

import numpy as np
import pytest

import oracle
from llambda_amd import ggml
from llambda_amd.llama import HipLlamaSession, LlamaConfig, LlamaError, synthetic_llama

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-3


def _kv(c, context=None):
    return np.zeros((c.layer_count, 2, c.kv_head_count, context or c.context, c.head_dim),
                    dtype=np.float32)


def _row_abs_sum(t, rows, cols, xin):
    w = oracle.dequantize(t[0], t[1], rows * cols).reshape(rows, cols).astype(np.float64)
    return np.abs(w) @ np.abs(xin.astype(np.float64))


def _check_logits(got, ref, what):
    err = np.max(np.abs(got.astype(np.float64) - ref)) / np.abs(ref).max()
    print(f"{what}: max |dlogit| / max |logit| = {err:.2e}", flush=True)
    assert err < LOGIT_TOL, what
    assert np.argmax(got) == np.argmax(ref) or \
        abs(ref[np.argmax(got)] - ref.max()) < LOGIT_TOL * np.abs(ref).max()


def _check_slot(sess, w, kv, layer, pos, token=None):
    """Layer-0 cache slot against the oracle's within the projection bound."""
    c = w.config
    k, v = sess.read_kv(layer, pos, 1)
    rk, rv = kv[layer, 0, :, pos], kv[layer, 1, :, pos]
    if layer == 0 and token is not None:
        H = c.hidden
        rb = ggml.row_bytes(w.token_embd[0], H)
        x = oracle.dequantize(w.token_embd[0], w.token_embd[1][token * rb:(token + 1) * rb], H)
        xin = oracle.rms_norm(x, w.layers[0].attn_norm, c.norm_epsilon)
        nk = c.kv_head_count * c.head_dim
        sk = _row_abs_sum(w.layers[0].attn_k, nk, H, xin).reshape(c.kv_head_count, c.head_dim)
        sv = _row_abs_sum(w.layers[0].attn_v, nk, H, xin).reshape(c.kv_head_count, c.head_dim)
        # a rotated pair mixes two rows: bound by the pair's sum
        pair = sk.reshape(c.kv_head_count, -1, 2).sum(axis=2).repeat(2, axis=1)
        assert np.all(np.abs(v[:, 0] - rv) <= 1e-4 * sv + 1e-30)
        assert np.all(np.abs(k[:, 0] - rk) <= 1e-4 * pair + 1e-30)
    else:
        scale = max(np.abs(rk).max(), np.abs(rv).max())
        assert np.max(np.abs(k[:, 0] - rk)) < 1e-3 * scale
        assert np.max(np.abs(v[:, 0] - rv)) < 1e-3 * scale


CONFIGS = {
    # name: (config, extra synthetic_llama arguments)
    "g4d128": (LlamaConfig(hidden=512, layer_count=2, head_count=4, kv_head_count=1, ffn=1024,
                           vocab=96, rope_dimension=128, context=300), {}),
    "g2d64": (LlamaConfig(hidden=256, layer_count=2, head_count=4, kv_head_count=2, ffn=512,
                          vocab=80, rope_dimension=64, context=40), {"rope_factors": False}),
    "g8d128_qk_types_differ": (LlamaConfig(hidden=1024, layer_count=1, head_count=8,
                                           kv_head_count=1, ffn=768, vocab=64,
                                           rope_dimension=96, context=130),
                               {"attn_v_type": ggml.Q4_K, "ffn_down_type": ggml.Q4_K}),
    "g1d128": (LlamaConfig(hidden=256, layer_count=1, head_count=2, kv_head_count=2, ffn=256,
                           vocab=40, rope_dimension=128, context=20), {"output_type": ggml.Q4_K}),
}


@pytest.mark.parametrize("name", list(CONFIGS))
def test_llama_steps_from_empty_cache(hip, name):
    c, extra = CONFIGS[name]
    rng = np.random.default_rng(sum(name.encode()))
    w = synthetic_llama(rng, c, **extra)
    if name == "g8d128_qk_types_differ":
        # q and k of different types: separate q and k projections
        L = w.layers[0]
        from llambda_amd import synthetic
        L.attn_k = (ggml.Q6_K, synthetic.q6_k(rng, c.kv_head_count * c.head_dim, c.hidden))
    sess = HipLlamaSession(w)
    kv = _kv(c)
    try:
        for pos, token in enumerate([3, 17, 0, c.vocab - 1]):
            print(f"{name}: step {pos} token {token}", flush=True)
            got = sess.step(token, pos)
            ref = oracle.llama_step(w, kv, token, pos, threads=8)
            _check_logits(got, ref, f"{name} pos {pos}")
            _check_slot(sess, w, kv, 0, pos, token)
            _check_slot(sess, w, kv, c.layer_count - 1, pos)
    finally:
        sess.close()


@pytest.mark.parametrize("prefill", [62, 63, 64, 127, 128, 129, 290])
def test_llama_step_over_prefilled_cache(hip, prefill):
    """Cache slots 0..prefill-1 written from the host; the step at `prefill`
    attends over 1 to 5 chunks of 64 slots (the cross-chunk combine, its
    quarters of the chunks partly empty)."""
    c, _ = CONFIGS["g4d128"]
    rng = np.random.default_rng(prefill)
    w = synthetic_llama(rng, c)
    sess = HipLlamaSession(w)
    kv = _kv(c)
    kv[:, :, :, :prefill] = rng.normal(size=kv[:, :, :, :prefill].shape)
    try:
        for layer in range(c.layer_count):
            sess.write_kv(layer, 0, kv[layer, 0, :, :prefill], kv[layer, 1, :, :prefill])
        k, v = sess.read_kv(1, 0, prefill)
        assert np.array_equal(k, kv[1, 0, :, :prefill]) and np.array_equal(v, kv[1, 1, :, :prefill])
        got = sess.step(7, prefill)
        ref = oracle.llama_step(w, kv, 7, prefill, threads=8)
        _check_logits(got, ref, f"prefill {prefill}")
        _check_slot(sess, w, kv, 0, prefill, 7)
    finally:
        sess.close()


def test_llama_step_over_a_long_prefilled_cache(hip):
    """8300 cached slots: 130 chunks of 64, whose combine quarters of 33
    chunks take a second round of loads."""
    c = dataclasses.replace(CONFIGS["g4d128"][0], context=8400)
    prefill = 8300
    rng = np.random.default_rng(8300)
    w = synthetic_llama(rng, c)
    sess = HipLlamaSession(w)
    kv = _kv(c)
    kv[:, :, :, :prefill] = rng.normal(size=kv[:, :, :, :prefill].shape)
    try:
        for layer in range(c.layer_count):
            sess.write_kv(layer, 0, kv[layer, 0, :, :prefill], kv[layer, 1, :, :prefill])
        got = sess.step(7, prefill)
        ref = oracle.llama_step(w, kv, 7, prefill, threads=8)
        _check_logits(got, ref, f"prefill {prefill}")
    finally:
        sess.close()


def test_llama_graph_replay_matches_eager(hip):
    """step_device replays one captured graph for every position; its logits
    equal the eager step's bit for bit (same kernels, same order), with eager
    steps and host synchronisations between the replays."""
    c, _ = CONFIGS["g4d128"]
    rng = np.random.default_rng(11)
    w = synthetic_llama(rng, c)
    sess = HipLlamaSession(w)
    try:
        for pos, token in enumerate([5, 9, 1, 44, 2]):
            eager = sess.step(token, pos)
            sess.step_device(token, pos, graph=True)
            assert np.array_equal(eager, sess.logits()), pos
            sess.step_device(token, pos, graph=False)
            assert np.array_equal(eager, sess.logits()), pos
        # two replays back to back, then a different position
        sess.step_device(3, 5, graph=True)
        sess.step_device(4, 6, graph=True)
        replay = sess.logits()
        assert np.array_equal(replay, sess.step(4, 6))
    finally:
        sess.close()


def test_llama_step_then_sample_on_device(hip):
    """step_device into the session's logits, then the sampler reads them on
    the device: the oracle's token for the same logits."""
    from llambda_amd.sampling import HipSampler
    c, _ = CONFIGS["g4d128"]
    w = synthetic_llama(np.random.default_rng(14), c)
    sess = HipLlamaSession(w)
    sampler = HipSampler(c.vocab)
    rng = np.random.default_rng(15)
    history = []
    try:
        token = 1
        for pos in range(6):
            sess.step_device(token, pos, graph=True)
            roll = float(np.float32(rng.random()))
            kw = dict(history=history, top_k=40, top_p=0.9, temperature=0.8, random_value=roll)
            got = sampler.sample_session(sess, **kw)
            assert got == oracle.sample_token(sess.logits(), **kw), pos
            history.append(got)
            token = got
    finally:
        sampler.close()
        sess.close()


def test_steps_on_caller_streams_are_ordered(hip):
    """Steps enqueued on two different caller streams, each followed at once
    by a device-side sample of the session's logits: every step waits for the
    previous one and the sampler for the last, so the tokens and logits are
    those of the same steps run synchronously on a second session."""
    import torch

    from llambda_amd.sampling import HipSampler
    c, _ = CONFIGS["g4d128"]
    w = synthetic_llama(np.random.default_rng(17), c)
    a, b = HipLlamaSession(w), HipLlamaSession(w)
    sampler = HipSampler(c.vocab)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    try:
        token = 3
        for pos in range(8):
            st = streams[pos % 2].cuda_stream
            a.step_device(token, pos, stream=st, graph=bool(pos % 3))
            kw = dict(top_k=40, top_p=0.9, temperature=1.0, random_value=0.37)
            got = sampler.sample_session(a, **kw)
            ref = b.step(token, pos)
            assert np.array_equal(a.logits(), ref), pos
            assert got == oracle.sample_token(ref, **kw), pos
            token = got
    finally:
        sampler.close()
        a.close()
        b.close()


def test_llama_from_gguf_file(hip, tmp_path):
    """A model written to a GGUF file, mapped, parsed and uploaded straight
    from the mapping (the file is closed before the steps run)."""
    from llambda_amd.gguf import GgufFile, load_llama, save_llama
    c, _ = CONFIGS["g4d128"]
    w = synthetic_llama(np.random.default_rng(16), c)
    path = str(tmp_path / "model.gguf")
    save_llama(path, w)
    with GgufFile(path) as f:
        sess = HipLlamaSession(load_llama(f, context=c.context))
    kv = _kv(c)
    try:
        for pos, token in enumerate([2, 7, 11]):
            got = sess.step(token, pos)
            ref = oracle.llama_step(w, kv, token, pos, threads=8)
            _check_logits(got, ref, f"gguf pos {pos}")
    finally:
        sess.close()


def test_llama_8b_layer_shapes_at_4096(hip):
    """Two layers of the Llama-3.1-8B layout (hidden 4096, 32 query / 8 kv
    heads of 128, SwiGLU 14336, Q4_K_M mix, Llama-3.1 rotation factors) with
    the fp32 cache prefilled to 4096 slots ~ N(0, 1); the step at 4096."""
    c = LlamaConfig(hidden=4096, layer_count=2, head_count=32, kv_head_count=8, ffn=14336,
                    vocab=512, rope_dimension=128, context=4224)
    rng = np.random.default_rng(8)
    w = synthetic_llama(rng, c)
    sess = HipLlamaSession(w)
    kv = _kv(c)
    kv[:, :, :, :4096] = rng.normal(size=kv[:, :, :, :4096].shape)
    try:
        for layer in range(c.layer_count):
            sess.write_kv(layer, 0, kv[layer, 0, :, :4096], kv[layer, 1, :, :4096])
        got = sess.step(123, 4096)
        ref = oracle.llama_step(w, kv, 123, 4096, threads=16)
        _check_logits(got, ref, "8B layers at 4096")
        _check_slot(sess, w, kv, 0, 4096, 123)
        _check_slot(sess, w, kv, 1, 4096)
    finally:
        sess.close()


def _host_copy(w_dev):
    """Host LlamaWeights with the bytes of device-drawn weights."""
    from llambda_amd.llama import LlamaLayerWeights, LlamaWeights

    def h(t):
        return (t.type, t.owner.reshape(-1).cpu().numpy())

    layers = [LlamaLayerWeights(attn_norm=L.attn_norm, attn_q=h(L.attn_q), attn_k=h(L.attn_k),
                                attn_v=h(L.attn_v), attn_output=h(L.attn_output),
                                ffn_norm=L.ffn_norm, ffn_gate=h(L.ffn_gate), ffn_up=h(L.ffn_up),
                                ffn_down=h(L.ffn_down)) for L in w_dev.layers]
    return LlamaWeights(config=w_dev.config, token_embd=h(w_dev.token_embd),
                        output=h(w_dev.output), output_norm=w_dev.output_norm,
                        rope_factors=w_dev.rope_factors, layers=layers)


def test_llama31_8b_full_token_at_4096(hip):
    """The whole Llama-3.1-8B-layout token the benchmark times: 32 layers,
    the 128256-row Q6_K output head with output_norm fused, the fp32 cache
    prefilled to 4096 slots ~ N(0, 1), the step at 4096 -- against the
    oracle's step on the same bytes.  Every logit within 1e-4 of
    sum_i |w_ri h_i| of its row (h the oracle's input to the output rows: the
    north-star bound, with the 32 layers' own rounding inside it), plus the
    per-row bound of the layer-0 cache slot and the largest-logit check."""
    import os

    import torch

    from llambda_amd.llama import LLAMA31_8B, synthetic_llama_device

    from helpers import abs_dot_bound

    c = LLAMA31_8B
    context, pos, token = 4224, 4096, 4242
    print("full 8B token: drawing weights on the device", flush=True)
    w_dev = synthetic_llama_device(41, c, np.random.default_rng(41))
    sess = HipLlamaSession(w_dev, context=context)
    try:
        w = _host_copy(w_dev)
        del w_dev
        torch.cuda.empty_cache()
        kv = np.zeros((c.layer_count, 2, c.kv_head_count, context, c.head_dim), dtype=np.float32)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(42)
        for layer in range(c.layer_count):
            k = torch.randn((c.kv_head_count, pos, c.head_dim), device="cuda", generator=gen)
            v = torch.randn((c.kv_head_count, pos, c.head_dim), device="cuda", generator=gen)
            torch.cuda.synchronize()
            sess.write_kv_device(layer, 0, pos, k.data_ptr(), v.data_ptr())
            kv[layer, 0, :, :pos] = k.cpu().numpy()
            kv[layer, 1, :, :pos] = v.cpu().numpy()
        del k, v
        print("full 8B token: device step", flush=True)
        got = sess.step(token, pos)
        print("full 8B token: oracle step", flush=True)
        threads = min(16, os.cpu_count() or 1)
        ref, hidden = oracle.llama_step(w, kv, token, pos, threads=threads, return_hidden=True)
        _check_logits(got, ref, "full 8B token at 4096")
        bound = abs_dot_bound(w.output[0], w.output[1], c.vocab, c.hidden, hidden)
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        ratio = float(np.max(err / bound))
        print(f"full 8B token: max |dlogit| / sum|w h| = {ratio:.2e}", flush=True)
        assert ratio <= 1e-4, ratio
        _check_slot(sess, w, kv, 0, pos, token)
        _check_slot(sess, w, kv, c.layer_count - 1, pos)
    finally:
        sess.close()


def test_llama_session_errors(hip):
    c, _ = CONFIGS["g2d64"]
    w = synthetic_llama(np.random.default_rng(12), c, rope_factors=False)
    sess = HipLlamaSession(w)
    try:
        with pytest.raises(LlamaError, match="token id"):
            sess.step(c.vocab, 0)
        with pytest.raises(LlamaError, match="position"):
            sess.step(0, c.context)
        with pytest.raises(LlamaError, match="outside the context"):
            sess.read_kv(0, c.context - 1, 2)
    finally:
        sess.close()
    bad = LlamaConfig(hidden=256, layer_count=1, head_count=2, kv_head_count=2, ffn=256, vocab=8,
                      rope_dimension=128, context=8)
    w = synthetic_llama(np.random.default_rng(13), bad)
    w.layers[0].attn_q = (ggml.Q5_0, np.zeros(256 * 256 // 32 * 22, dtype=np.uint8))
    with pytest.raises(LlamaError, match="not supported by the decoder"):
        HipLlamaSession(w)
    w = synthetic_llama(np.random.default_rng(13), bad)
    blocks = w.layers[0].ffn_up[1].reshape(-1, 144).copy()
    blocks[3, 0:2] = np.array([0x00, 0x7C], dtype=np.uint8)  # d = +inf
    w.layers[0].ffn_up = (ggml.Q4_K, blocks.reshape(-1))
    with pytest.raises(LlamaError, match="Inf/NaN"):
        HipLlamaSession(w)
