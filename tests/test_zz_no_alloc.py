"""The MoE entry point that allocates nothing
(llambda_hip_moe_session_run_device_noalloc) against the device run with the
session's own scratch (llambda_hip_moe_session_run_device): the same kernels
in the same order, so the outputs are bit-identical.  Two calls in a row, the
second with a smaller input; then a batch beyond the scratch's maximum is
refused with an error before anything runs."""
import ctypes

import numpy as np
import pytest

from llambda_amd import ggml, native, synthetic
from llambda_amd.moe import HipMoeSession, synthetic_nemotron_h, synthetic_qwen3next

pytestmark = pytest.mark.gpu


def _noalloc(session, x_ptr, y_ptr, tokens, stream):
    return native.lib().llambda_hip_moe_session_run_device_noalloc(session.pointer, x_ptr, y_ptr,
                                                                   tokens, stream)


def _layer(variant, rng):
    """Layers and batch sizes that reach every pipeline on the carved array:
    one token (fused gating, down + combine), 16-pair chunks (at most 16
    pairs per expert on average), the wide pipeline (K-quant experts, more
    than 16 pairs per expert) and the group pipeline (32-weight block types,
    more than 16 pairs per expert: 300 tokens x 2 of 8 experts = 75), and a
    Nemotron-H layer with ffn_latent_down / ffn_latent_up."""
    if variant == "qwen3next":
        return synthetic_qwen3next(rng, hidden=1024, experts=64, top_k=6, ffn=256,
                                   shared_ffn=256), (40, 7)
    if variant == "nemotron":
        return synthetic_nemotron_h(rng, hidden=768, experts=32, top_k=4, ffn=320,
                                    shared_ffn=640), (33, 1)
    if variant == "latent":
        return synthetic_nemotron_h(rng, hidden=512, experts=8, top_k=2, ffn=288, shared_ffn=320,
                                    expert_type=ggml.Q8_0, down_type=ggml.Q5_0, latent_in=256,
                                    latent_out=192, latent_type=ggml.Q5_0), (300, 1)
    if variant == "wide":
        return synthetic_qwen3next(rng, hidden=512, experts=8, top_k=2, ffn=256,
                                   shared_ffn=256), (300, 120)
    return synthetic_nemotron_h(rng, hidden=512, experts=8, top_k=2, ffn=288, shared_ffn=320,
                                expert_type=ggml.Q8_0, down_type=ggml.Q5_0), (300, 90)


@pytest.mark.parametrize("variant", ["qwen3next", "nemotron", "wide", "group", "latent"])
def test_noalloc_matches_the_allocating_run(hip, variant):
    import torch
    rng = np.random.default_rng(70)
    layer, sizes = _layer(variant, rng)
    session = HipMoeSession(layer)
    stream = torch.cuda.Stream()
    try:
        for tokens in sizes:
            print(f"noalloc {variant}: {tokens} tokens", flush=True)
            x = torch.from_numpy(synthetic.activations(rng, tokens, layer.hidden)).cuda()
            y_ref = torch.empty_like(x)
            y = torch.full_like(x, float("nan"))
            torch.cuda.synchronize()
            session.run_device(x.data_ptr(), y_ref.data_ptr(), tokens, stream.cuda_stream)
            session.sync(stream.cuda_stream)
            assert _noalloc(session, x.data_ptr(), y.data_ptr(), tokens, stream.cuda_stream) == 0, \
                native.last_error()
            session.sync(stream.cuda_stream)
            assert torch.equal(y, y_ref), f"{variant} {tokens} tokens"
        # beyond the maximum: refused before anything is enqueued
        big = 4096
        x = torch.zeros((big, layer.hidden), device="cuda")
        y = torch.zeros_like(x)
        torch.cuda.synchronize()
        assert _noalloc(session, x.data_ptr(), y.data_ptr(), big, stream.cuda_stream) == -1
        assert "bytes of scratch" in native.last_error()
        assert torch.count_nonzero(y).item() == 0
        session.sync(stream.cuda_stream)
    finally:
        session.close()


def test_noalloc_reports_kernel_errors_through_sync(hip):
    """A NaN token (fewer than k selectable logits): the reference's error,
    reported by moe_session_sync; the next call starts from a clean flag."""
    import torch
    from llambda_amd.moe import MoeLayerInputError
    rng = np.random.default_rng(71)
    layer = synthetic_qwen3next(rng, hidden=256, experts=16, top_k=2, ffn=64, shared_ffn=64,
                                down_type=ggml.Q8_0)
    session = HipMoeSession(layer)
    try:
        x = torch.full((1, 256), float("nan"), device="cuda")
        y = torch.empty_like(x)
        torch.cuda.synchronize()
        assert _noalloc(session, x.data_ptr(), y.data_ptr(), 1, None) == 0
        with pytest.raises(MoeLayerInputError, match="Qwen3Next layer router produced"):
            session.sync()
        good = torch.from_numpy(synthetic.activations(rng, 2, 256)).cuda()
        y2 = torch.empty_like(good)
        ref = session.run(good.cpu().numpy())
        assert _noalloc(session, good.data_ptr(), y2.data_ptr(), 2, None) == 0
        session.sync()
        assert np.array_equal(y2.cpu().numpy(), ref)
    finally:
        session.close()


def test_noalloc_calls_on_two_streams_and_sessions_do_not_overlap(hip):
    """Two sessions, each on its own stream, enqueue no-allocation calls back
    to back without waiting: the calls share the GPU's scratch array, so the
    library orders them on the device, and every output equals that session's
    allocating run."""
    import torch
    rng = np.random.default_rng(72)
    layers = [synthetic_qwen3next(rng, hidden=512, experts=8, top_k=2, ffn=256, shared_ffn=256),
              synthetic_nemotron_h(rng, hidden=512, experts=8, top_k=2, ffn=288, shared_ffn=320,
                                   expert_type=ggml.Q8_0, down_type=ggml.Q5_0)]
    sessions = [HipMoeSession(layer) for layer in layers]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    try:
        plan = [(0, 300), (1, 250), (0, 64), (1, 300), (0, 1), (1, 17)]
        xs, ys, refs = [], [], []
        for i, tokens in plan:
            x = torch.from_numpy(synthetic.activations(rng, tokens, 512)).cuda()
            y_ref = torch.empty_like(x)
            sessions[i].run_device(x.data_ptr(), y_ref.data_ptr(), tokens, streams[i].cuda_stream)
            sessions[i].sync(streams[i].cuda_stream)
            xs.append(x)
            ys.append(torch.full_like(x, float("nan")))
            refs.append(y_ref)
        torch.cuda.synchronize()
        print("noalloc: six calls on two streams, no waits between them", flush=True)
        for (i, tokens), x, y in zip(plan, xs, ys):
            assert _noalloc(sessions[i], x.data_ptr(), y.data_ptr(), tokens,
                            streams[i].cuda_stream) == 0, native.last_error()
        for i in range(2):
            sessions[i].sync(streams[i].cuda_stream)
        for k, (y, y_ref) in enumerate(zip(ys, refs)):
            assert torch.equal(y, y_ref), f"call {k} {plan[k]}"
    finally:
        for s in sessions:
            s.close()
