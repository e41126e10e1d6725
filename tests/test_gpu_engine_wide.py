"""GPU tests of the decode engine at the production widths of the three
quantized models (model_config.h:77-102): Qwen3.5-9B Q8_0 (H 4096, I 12288),
Qwen3.8-27B Q4_0 (H 5120, I 17408, 24 query heads) and Qwen3.6-35B-A3B Q4_0
(256 experts, top 8, shared expert 512), with four layers (three DeltaNet,
one attention) and a small vocabulary, against the reference's own CPU
forward (engine.cpp:431-454, built from the reference sources into
oracle/_ref).  A prompt of 12 tokens runs as prefill chunks of 8 rows (a
chunk boundary inside it), then 4 decode steps; the logits after the prompt
and after every decode step must lie within 2e-4 + 2e-4 |reference|, the
bound of the reference's synthetic forward test (tests/metal_test.mm:121-124).
These widths take the staging paths the small models cannot reach: the norm
staging's second chunk (H 5120), SwiGLU staging over 384 and 544 blocks, the
32-lane Q4_0 rows of 160-block rows, six query heads per KV head, and the
256-expert decode MoE that adds into the residual.  The three reference
forwards (the slow part: about 0.4-1.8 s per token on one core) run in
parallel threads while the first test waits."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import oracle
import qwen3x_amd as q3x
from tests.engine_models import WIDE, wide_model
from tests.test_gpu_parity import _torch, dev, say

pytestmark = pytest.mark.gpu

PROMPT, DECODE, CHUNK = 12, 4, 8


def _reference(name):
    fields = WIDE[name]
    config, image, table = wide_model(fields, seed=fields["id"])
    rng = np.random.default_rng(300 + fields["id"])
    tokens = rng.integers(0, fields["V"], PROMPT + DECODE).astype(np.int32)
    want = oracle.ref_forward(fields, image, table, tokens)
    return config, image, tokens, want


@pytest.fixture(scope="module")
def references():
    if oracle.ref() is None:
        pytest.skip("reference build (oracle/_ref) absent")
    _torch()
    q3x.lib()  # loaded once, here, before the worker threads use it
    with ThreadPoolExecutor(len(WIDE)) as pool:
        yield {name: pool.submit(_reference, name) for name in sorted(WIDE)}


def _check(got, want, what):
    assert np.all(np.isfinite(got)), what
    diff = np.abs(got - want)
    bound = 2e-4 + 2e-4 * np.abs(want)
    worst = float((diff / bound).max())
    say(f"  {what}: worst |delta|/bound = {worst:.3g}")
    assert np.all(diff <= bound), f"{what}: worst {diff.max()} at {diff.argmax()}"


@pytest.mark.parametrize("name", sorted(WIDE))
def test_wide_prefill_then_decode_match_the_reference_forward(name, references):
    torch = _torch()
    say(f"engine {name}: waiting for the reference forward ({oracle.ref_variant()[0]} build)")
    config, image, tokens, want = references[name].result()
    say(f"engine {name}: prefill {PROMPT} (chunk {CHUNK}) + decode {DECODE}")
    weights = dev(image)
    with q3x.Engine(config, weights, context=len(tokens), chunk=CHUNK) as engine:
        engine.forward(tokens[:PROMPT])
        _check(engine.logits(), want[PROMPT - 1], "prefill")
        for i in range(PROMPT, len(tokens)):
            engine.forward(tokens[i:i + 1])
            _check(engine.logits(), want[i], f"decode {i}")
    del weights
    torch.cuda.empty_cache()
