"""The product decode-step driver (xn_amd.decode.DecodeStep) at config 5's
layer shapes: hidden 4096, 8 kv heads of 128 (k/v 4096 -> 1024), FFN 14336,
vocab 128256, Q4_K attention and gate/up, Q6_K down and lm_head; two layers,
batch 1 and 16, run eagerly and as a replayed graph (cuda_backend/mod.rs:236-300).

Every product of the step is checked against the AVX2 restatement of xn's
CPU path on the very activation the device fed it (its input buffer after
the run), so one product's tolerance does not compound into the next check.
Bars as in test_gpu_parity."""
import os

import numpy as np
import pytest
import torch

from tests.test_gpu_parity import assert_close

pytestmark = pytest.mark.gpu

SEED = 1234567


@pytest.fixture(scope="module")
def checker(orc):
    orc.cpu_pool_init(min(16, os.cpu_count() or 1))
    return orc


@pytest.fixture(scope="module")
def weights(dev):
    from xn_amd.decode import DecoderWeights

    g = torch.Generator(device=dev).manual_seed(SEED)
    return DecoderWeights.random(2, 4096, 1024, 14336, 128256, dev, generator=g)


def check_products(checker, step):
    blocks = {}

    def host_blocks(qt):
        if id(qt) not in blocks:
            blocks[id(qt)] = np.frombuffer(qt.data(), dtype=np.uint8)
        return blocks[id(qt)]

    for name, w, x, y in step.products():
        xh = x.cpu().numpy().astype(np.float32)
        got = y.cpu().numpy()
        if isinstance(w, tuple):  # gate/up with the SiLU gate (llama.rs:258-264)
            g = checker.cpu_matmul(int(w[0].dtype()), xh, host_blocks(w[0]), w[0].shape()[0]).astype(np.float64)
            u = checker.cpu_matmul(int(w[1].dtype()), xh, host_blocks(w[1]), w[1].shape()[0])
            want = g / (1.0 + np.exp(0.0 - g)) * u
        else:
            want = checker.cpu_matmul(int(w.dtype()), xh, host_blocks(w), w.shape()[0])
        assert np.isfinite(got).all(), name
        assert_close(got, want, f"decode step b={step.b} {name}")


@pytest.mark.parametrize("batch", [1, 16])
def test_decode_step_parity(checker, weights, dev, batch):
    from xn_amd.decode import DecodeStep

    step = DecodeStep(weights, batch, dev)
    x0 = torch.from_numpy(np.random.default_rng(SEED + batch).normal(0, 1, (batch, 4096)).astype(np.float32))
    step.x.copy_(x0.to(dev))
    step.run()
    torch.cuda.synchronize()
    check_products(checker, step)
    eager = {name: y.clone() for name, _, _, y in step.products()}

    # the captured graph replays the same products: clear every output, replay
    # twice with eager work in between, and compare with the eager results
    stream = torch.cuda.Stream(dev)
    step.capture(stream)
    for rep in range(2):
        for _, _, _, y in step.products():
            y.fill_(float("nan"))
        torch.cuda.synchronize()
        step.replay()
        stream.synchronize()
        for name, _, _, y in step.products():
            assert torch.equal(y, eager[name]), f"replay {rep}: {name} differs from the eager run"


def test_decode_step_glue_hooks(dev):
    """Glue runs at its three points per layer and its outputs feed the next
    product (here: attention output = 0.5 q, residual x_next = x + down)."""
    from xn_amd.decode import DecoderWeights, DecodeStep

    g = torch.Generator(device=dev).manual_seed(SEED + 3)
    w = DecoderWeights.random(2, 256, 256, 512, 1000, dev, generator=g)
    seen = []

    def glue(point, layer, b):
        seen.append((point, layer))
        if point == "attention":
            torch.mul(b["q"], 0.5, out=b["attn"])
        elif point == "post_mlp":
            torch.add(b["x"], b["down"], out=b["x_next"])

    step = DecodeStep(w, 3, dev, glue=glue)
    step.x.normal_(generator=g)
    step.run()
    torch.cuda.synchronize()
    assert seen == [(p, l) for l in range(2) for p in ("attention", "post_attention", "post_mlp")]
    for l, b in enumerate(step.bufs):
        assert torch.equal(b["attn"], b["q"] * 0.5)
        assert torch.equal(b["x_next"], b["x"] + b["down"])
    ref = torch.empty_like(step.logits)
    w.lm_head.matmul_t((3, 256, 1000), step.bufs[-1]["x_next"], ref)
    torch.cuda.synchronize()
    assert torch.equal(ref, step.logits)


def test_decode_step_rejects_bad_shapes(dev):
    from xn_amd import XnqError
    from xn_amd.decode import DecoderWeights, DecodeStep

    g = torch.Generator(device=dev).manual_seed(SEED + 4)
    w = DecoderWeights.random(1, 256, 256, 512, 300, dev, generator=g)
    w.layers[0].o = w.layers[0].gate  # (512, 256) where (256, 256) is expected
    with pytest.raises(XnqError):
        DecodeStep(w, 1, dev)
