"""GPU tests of the decode engine (q3x_hip_engine_*) against the reference's
own CPU forward (engine.cpp:431-454, built from the reference sources into
oracle/_ref) on small synthetic models with the real head sizes: logits after
every token within 2e-4 + 2e-4 |reference|, the bound of the reference's own
synthetic forward test (tests/metal_test.mm:121-124).  The reference forward
runs here and on the GPU box from the built library; with it absent these
tests skip."""
import numpy as np
import pytest

import oracle
import qwen3x_amd as q3x
from tests.engine_models import CONFIGS, synthetic_model
from tests.test_gpu_parity import _torch, dev, say

pytestmark = pytest.mark.gpu


def _need_ref():
    if oracle.ref() is None:
        pytest.skip("reference build (oracle/_ref) absent")


def _bound(want):
    return 2e-4 + 2e-4 * np.abs(want)


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_engine_logits_match_the_reference_forward(name):
    _need_ref()
    _torch()
    fields = CONFIGS[name]
    config, image, table = synthetic_model(fields, seed=fields["id"])
    rng = np.random.default_rng(100 + fields["id"])
    tokens = rng.integers(0, fields["V"], 12).astype(np.int32)
    want = oracle.ref_forward(fields, image, table, tokens)
    weights = dev(image)
    say(f"engine {name}: {len(tokens)} tokens, reference {oracle.ref_variant()[0]} build")
    with q3x.Engine(config, weights, context=len(tokens)) as engine:
        for i, tok in enumerate(tokens):
            engine.forward([tok])
            got = engine.logits()
            assert np.all(np.isfinite(got)), i
            diff = np.abs(got - want[i])
            assert np.all(diff <= _bound(want[i])), f"token {i}: worst {diff.max()} at {diff.argmax()}"
        assert engine.position == len(tokens)


@pytest.mark.parametrize("name,prompt,chunk", [("dense_q8", 40, 0), ("dense_q4", 530, 256), ("moe_q4", 300, 0),
                                               ("moe_q8_tied", 64, 48), ("gqa8_q8", 100, 0), ("dense_q8", 333, 100),
                                               ("gqa8_q8", 2100, 2048), ("narrow_q4", 300, 128), ("odd_q8", 300, 0),
                                               ("gqa8_q8", 4200, 0), ("dense_q8", 8300, 0)])
def test_prefill_then_decode_match_the_reference_forward(name, prompt, chunk):
    # A forward of many tokens runs them as prefill chunks (GEMMs, the delta
    # rule in 32-token chunks on the matrix cores -- token by token for the
    # odd head sizes -- attention on the matrix cores); its logits, and
    # those of the decode steps that follow, against
    # the reference's token-by-token forward.  Chunks of 256, 48 and 100 rows
    # put chunk boundaries inside the prompts, and tiles of 32 query rows
    # end partly filled; 2100 tokens cross a 2048-row chunk with
    # every query tile spanning up to 66 key blocks.  At 4200 (8 query heads
    # per KV head) and 8300 (2) positions, each of a decode step's 128
    # position ranges is longer than one block of the decode attention (32 /
    # 64 positions), so its online softmax rescales across blocks.
    _need_ref()
    _torch()
    fields = CONFIGS[name]
    config, image, table = synthetic_model(fields, seed=fields["id"] + 20)
    rng = np.random.default_rng(200 + fields["id"])
    tokens = rng.integers(0, fields["V"], prompt + 4).astype(np.int32)
    want = oracle.ref_forward(fields, image, table, tokens)
    weights = dev(image)
    say(f"engine {name}: prefill {prompt} (chunk {chunk}) + decode 4")
    with q3x.Engine(config, weights, context=len(tokens), chunk=chunk) as engine:
        engine.forward(tokens[:prompt])
        got = engine.logits()
        diff = np.abs(got - want[prompt - 1])
        assert np.all(diff <= _bound(want[prompt - 1])), f"prefill: worst {diff.max()}"
        for i in range(prompt, len(tokens)):
            engine.forward(tokens[i:i + 1])
            diff = np.abs(engine.logits() - want[i])
            assert np.all(diff <= _bound(want[i])), f"decode {i}: worst {diff.max()}"


def test_checkpoint_reset_and_errors():
    _torch()
    fields = CONFIGS["moe_q4"]
    config, image, _ = synthetic_model(fields, seed=9)
    rng = np.random.default_rng(10)
    prompt = rng.integers(0, fields["V"], 5).astype(np.int32)
    cont = rng.integers(0, fields["V"], 3).astype(np.int32)
    weights = dev(image)
    say("engine checkpoint / reset")
    with q3x.Engine(config, weights, context=8) as e:
        e.forward(prompt)
        first = e.logits()
        e.checkpoint_save()
        e.forward(cont)
        after = e.logits()
        e.checkpoint_restore()
        assert e.position == 5
        assert np.array_equal(e.logits().view(np.uint32), first.view(np.uint32))
        e.forward(cont)
        assert np.array_equal(e.logits().view(np.uint32), after.view(np.uint32))
        e.reset()
        assert e.position == 0
        e.forward(prompt)
        assert np.array_equal(e.logits().view(np.uint32), first.view(np.uint32))
        # context exhausted / bad tokens: rejected, nothing run
        with pytest.raises(q3x.Q3xHipError):
            e.forward(np.zeros(4, np.int32))
        with pytest.raises(q3x.Q3xHipError):
            e.forward([fields["V"]])
        assert e.position == 5
        # a rejected call leaves the engine usable (it is not a failed forward)
        e.forward(cont)
        assert e.position == 8
        assert np.array_equal(e.logits().view(np.uint32), after.view(np.uint32))
