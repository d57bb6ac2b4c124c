"""The synchronous host-pointer entry points (the calls the Lisp adapter
makes: llambda_hip_session_run[_batch], llambda_hip_moe_session_run) against
the device-pointer runs of the same kernels.

The host-pointer runs stage the input through pinned memory and, for one
token, let the final kernel store its rows straight into mapped host memory
(the MoE's final launch also stores the run's error word there); larger
batches copy the rows back.  The kernels are the same, so the results must be
equal bit for bit -- including a single token after the staging has grown for
a larger batch, and a run that reports a reference error followed by a
good one."""
import numpy as np
import pytest
import torch

from llambda_amd import ggml, synthetic
from llambda_amd.hip_backend import HipBackendError, make_hip_session_packed
from llambda_amd.moe import HipMoeSession, MoeLayerInputError, synthetic_qwen3next

pytestmark = pytest.mark.gpu


def _device_gemv(session, x, rows):
    xd = torch.from_numpy(np.ascontiguousarray(x)).to("cuda")
    yd = torch.empty((x.shape[0], rows), device="cuda", dtype=torch.float32)
    session.run_device(xd.data_ptr(), yd.data_ptr(), x.shape[0])
    torch.cuda.synchronize()
    return yd.cpu().numpy()


@pytest.mark.parametrize("type_tag", [ggml.Q4_K, ggml.Q6_K, ggml.Q8_0])
def test_gemv_host_runs_equal_device_runs(hip, type_tag):
    rows, columns = 777, 4096
    rng = np.random.default_rng(50 + type_tag)
    w = synthetic.packed(type_tag, rng, rows, columns)
    s = make_hip_session_packed(w, type_tag, rows, columns)
    try:
        for batch in (1, 4, 1, 7, 1, 2):
            x = synthetic.activations(rng, batch, columns)
            if batch == 1:
                y = np.empty(rows, dtype=np.float32)
                s.run_into(y, x[0])
                y = y[None, :]
            else:
                y = np.empty((batch, rows), dtype=np.float32)
                s.run_batch_into(y, x, batch)
            np.testing.assert_array_equal(y, _device_gemv(s, x, rows), err_msg=f"batch {batch}")
    finally:
        s.close()


def test_moe_host_runs_equal_device_runs(hip):
    rng = np.random.default_rng(60)
    layer = synthetic_qwen3next(rng, hidden=512, experts=32, top_k=4, ffn=256, shared_ffn=256)
    s = HipMoeSession(layer)
    try:
        for tokens in (1, 5, 1, 9, 1):
            x = synthetic.activations(rng, tokens, layer.hidden)
            if tokens == 1:
                y = np.empty(layer.hidden, dtype=np.float32)
                s.run_into(y, x[0])
                y = y[None, :]
            else:
                y = s.run(x)
            xd = torch.from_numpy(x).to("cuda")
            yd = torch.empty_like(xd)
            s.run_device(xd.data_ptr(), yd.data_ptr(), tokens)
            s.sync()
            np.testing.assert_array_equal(y, yd.cpu().numpy(), err_msg=f"{tokens} tokens")
    finally:
        s.close()


def test_moe_host_run_error_word_then_good_run(hip):
    """A NaN token reports the reference's router error (its own input error,
    status -2: non-positive top-k weight sum, llambda.lisp:5373) through the
    error word stored by the final launch; the flag is cleared, and the next
    one-token run succeeds and matches the device-pointer run."""
    rng = np.random.default_rng(61)
    layer = synthetic_qwen3next(rng, hidden=256, experts=16, top_k=2, ffn=256, shared_ffn=256)
    s = HipMoeSession(layer)
    try:
        bad = np.full(layer.hidden, np.nan, dtype=np.float32)
        with pytest.raises(MoeLayerInputError, match="router produced non-positive top-k weight sum"):
            s.run_into(np.empty(layer.hidden, dtype=np.float32), bad)
        x = synthetic.activations(rng, 1, layer.hidden)
        y = np.empty(layer.hidden, dtype=np.float32)
        s.run_into(y, x[0])
        assert np.isfinite(y).all()
        xd = torch.from_numpy(x).to("cuda")
        yd = torch.empty_like(xd)
        s.run_device(xd.data_ptr(), yd.data_ptr(), 1)
        s.sync()
        np.testing.assert_array_equal(y, yd.cpu().numpy()[0])
    finally:
        s.close()
