"""GPT-2 medium shapes through libtinyinfer_llm.so: hidden 1024, 16 heads x 64,
MLP 4096, vocab 50257, on a 2-layer synthetic INT8 artifact.

K = 1024 is the widest hidden size whose decode GEMVs take the LayerNorm
prologue, and 16 K chunks of the packed layout: the LM head at 17..32 rows runs
the wide GEMV over P32 activations at 16 chunks, at 1..16 rows the 4-wave
packed GEMV.  Against the CPU oracle (restating reference llm/src/runtime.cu):
logits within atol 5e-2 after a ragged 32-request prefill and decode steps; a
request's logits bit-identical alone and inside the 32-request batch (the two
head kernels sum K in one order); greedy runs of 20 requests (two decode lanes)
equal to each request decoded alone.

With 18 layers the INT8 decode weights (278 MB) exceed what the second decode
lane needs to find in the 256 MiB Infinity Cache, so a context decodes 17..32
requests in one lane: the step's LM head is then the wide GEMV over 32 P32 rows,
leaving per-workgroup argmax partials for the step's greedy feed.  Greedy tokens
of 24 requests together equal each request decoded alone (one row, the packed
GEMV head), and two decode steps' logits match the oracle.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

MEDIUM_2L = {"layers": 2, "heads": 16, "hidden": 1024, "vocab": 50257, "capacity": 1024,
             "gelu": "gelu_new", "layer_norm_eps": 1e-5}


def say(*args):
    print("[case]", *args, flush=True)


def logits_of(result):
    return np.frombuffer(result["logits"], dtype=np.float32).reshape(result["shape"]).copy()


@pytest.fixture(scope="module")
def artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import write_synthetic
    say("writing 2-layer GPT-2 medium-shaped synthetic artifact")
    return write_synthetic(tmp_path_factory.mktemp("gpt2m2"), MEDIUM_2L, seed=13)


@pytest.fixture(scope="module")
def model(artifact):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    say("creating native medium-shaped model")
    with NativeModel(LLM_LIB, artifact, max_batch=32, cache_slots=34, capacity=128) as m:
        yield m


@pytest.fixture(scope="module")
def cpu_model(artifact):
    from tinyinfer_amd.artifact import load_tensors
    manifest, tensors = load_tensors(artifact)
    m = oracle.Gpt2(tensors, manifest["architecture"], slots=34, capacity=128)
    yield m
    m.close()


def prompts_of(seed, count, lo=1, hi=40):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, 50257, int(n)).tolist() for n in rng.integers(lo, hi, count)]


def test_medium_logits_match_oracle_at_32_rows(model, cpu_model):
    prompts = prompts_of(3, 32)
    slots = list(range(32))
    say("medium: 32-request prefill and decode vs oracle")
    model.reset_all()
    for s in slots:
        cpu_model.reset(s)
    gpu = logits_of(model.forward(slots, prompts))
    cpu, nxt = cpu_model.forward(slots, prompts)
    print(f"medium prefill max |logit diff| {np.abs(gpu - cpu).max():.3g}")
    assert np.abs(gpu - cpu).max() <= 5e-2
    for _ in range(2):  # 32-row decode: LN-prologue GEMVs at K = 1024, the wide head at 16 chunks
        step = [[int(t)] for t in nxt]
        gpu = logits_of(model.forward(slots, step))
        cpu, nxt = cpu_model.forward(slots, step)
        print(f"medium decode max |logit diff| {np.abs(gpu - cpu).max():.3g}")
        assert np.abs(gpu - cpu).max() <= 5e-2
    model.reset_all()


def test_medium_request_alone_equals_batched(model):
    prompts = prompts_of(4, 32)
    say("medium: a request alone vs inside 32 requests")
    model.reset_all()
    batched = [logits_of(model.forward(list(range(32)), prompts))]
    for tok in (7, 50000):
        batched.append(logits_of(model.forward(list(range(32)), [[tok]] * 32)))
    for i in (0, 13, 31):
        model.reset(33)
        alone = logits_of(model.forward([33], [prompts[i]]))[0]
        assert np.array_equal(alone, batched[0][i]), f"prefill, request {i}"
        for step, tok in enumerate((7, 50000), start=1):
            alone = logits_of(model.forward([33], [[tok]]))[0]
            assert np.array_equal(alone, batched[step][i]), f"decode step {step}, request {i}"
    model.reset_all()


def test_medium_greedy_lanes_match_alone(model):
    prompts = prompts_of(5, 20, 3, 30)
    say("medium: 20-request greedy (two decode lanes) vs each request alone")
    model.reset_all()
    together = model.greedy(prompts, 8)["tokens"]
    for i in (0, 9, 16, 19):
        model.reset_all()
        alone = model.greedy([prompts[i]], 8, slots=[33])["tokens"][0]
        assert alone == together[i], f"request {i}"
    model.reset_all()


@pytest.fixture(scope="module")
def deep_artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import write_synthetic
    say("writing 18-layer GPT-2 medium-shaped synthetic artifact")
    return write_synthetic(tmp_path_factory.mktemp("gpt2m18"), dict(MEDIUM_2L, layers=18), seed=17)


def test_medium_one_lane_greedy_wide_head_matches_alone_and_oracle(deep_artifact):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.artifact import load_tensors
    from tinyinfer_amd.runtime import NativeModel
    prompts = prompts_of(6, 24, 2, 24)
    with NativeModel(LLM_LIB, deep_artifact, max_batch=32, cache_slots=34, capacity=64) as m:
        say("medium 18 layers: 24-request greedy in one lane vs each request alone")
        together = m.greedy(prompts, 6)["tokens"]
        for i in (0, 11, 23):
            m.reset_all()
            alone = m.greedy([prompts[i]], 6, slots=[33])["tokens"][0]
            assert alone == together[i], f"request {i}"
        say("medium 18 layers: 24-row decode logits vs oracle")
        m.reset_all()
        slots = list(range(24))
        gpu = logits_of(m.forward(slots, prompts))
        manifest, tensors = load_tensors(deep_artifact)
        cpu = oracle.Gpt2(tensors, manifest["architecture"], slots=24, capacity=64)
        try:
            ref, nxt = cpu.forward(slots, prompts)
            print(f"medium-18 prefill max |logit diff| {np.abs(gpu - ref).max():.3g}")
            assert np.abs(gpu - ref).max() <= 5e-2
            for _ in range(2):
                step = [[int(t)] for t in nxt]
                gpu = logits_of(m.forward(slots, step))
                ref, nxt = cpu.forward(slots, step)
                print(f"medium-18 decode max |logit diff| {np.abs(gpu - ref).max():.3g}")
                assert np.abs(gpu - ref).max() <= 5e-2
        finally:
            cpu.close()
