"""GPT-2 small from an fp16-precision artifact through libtinyinfer_llm.so: the
linears and the tied head stay fp16 (the reference runtime's other precision,
reference llm/src/runtime.cu:97-113, which runs them through ti_v2_gemm_ex_f16),
against the CPU oracle fed the same fp16 weights.  Logits within atol 5e-2 after
a ragged prefill and across decode steps (graph and eager), greedy tokens
identical or diverging only at near-ties (oracle gap at most 1e-2), and the
captured decode graph equal to the eager path bit for bit."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def say(*args):
    print("[case]", *args, flush=True)


def logits_of(result):
    return np.frombuffer(result["logits"], dtype=np.float32).reshape(result["shape"]).copy()


@pytest.fixture(scope="module")
def artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import GPT2_SMALL, write_synthetic
    say("writing GPT-2 small fp16-precision synthetic artifact")
    return write_synthetic(tmp_path_factory.mktemp("gpt2s16"), GPT2_SMALL, seed=21, precision="fp16")


@pytest.fixture(scope="module")
def cpu_model(artifact):
    from tinyinfer_amd.artifact import load_tensors
    manifest, tensors = load_tensors(artifact)
    assert manifest["precision"] == "fp16"
    m = oracle.Gpt2(tensors, manifest["architecture"], slots=9, capacity=128)
    yield m
    m.close()


@pytest.fixture(scope="module")
def model(artifact):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    say("creating native fp16-precision model")
    with NativeModel(LLM_LIB, artifact, max_batch=8, cache_slots=9, capacity=128) as m:
        yield m


def test_fp16_artifact_logits_match_oracle(model, cpu_model):
    rng = np.random.default_rng(31)
    prompts = [rng.integers(0, 50257, n).tolist() for n in (40, 3, 17, 1, 64)]
    slots = list(range(len(prompts)))
    say("fp16 artifact: prefill and decode logits vs oracle")
    model.reset_all()
    for s in slots:
        cpu_model.reset(s)
    gpu = logits_of(model.forward(slots, prompts))
    cpu, nxt = cpu_model.forward(slots, prompts)
    print(f"fp16 prefill max |logit diff| {np.abs(gpu - cpu).max():.3g}")
    assert np.abs(gpu - cpu).max() <= 5e-2
    for graph in (True, False, True):  # captured decode graph and the eager path
        step = [[int(t)] for t in nxt]
        gpu = logits_of(model.forward(slots, step, return_next=graph))
        cpu, nxt = cpu_model.forward(slots, step)
        print(f"fp16 decode ({'graph' if graph else 'eager'}) max |logit diff| {np.abs(gpu - cpu).max():.3g}")
        assert np.abs(gpu - cpu).max() <= 5e-2
    model.reset_all()


def test_fp16_artifact_greedy_matches_oracle(model, cpu_model):
    rng = np.random.default_rng(32)
    prompts = [rng.integers(0, 50257, 32).tolist() for _ in range(8)]
    new = 32
    say("fp16 artifact: greedy vs oracle")
    model.reset_all()
    gpu = model.greedy(prompts, new)["tokens"]
    for s in range(8):
        cpu_model.reset(s)
    cpu = cpu_model.greedy(list(range(8)), prompts, new)
    gaps = {}
    for b, (g, c) in enumerate(zip(gpu, cpu)):
        i = next((i for i, (x, y) in enumerate(zip(g, c)) if x != y), None)
        if i is not None:
            cpu_model.reset(8)
            lg, _ = cpu_model.forward([8], [prompts[b] + c[:i]])
            gaps[b] = (i, float(lg[0][c[i]] - lg[0][g[i]]))
    print(f"fp16 greedy: {8 - len(gaps)}/8 identical over {new} tokens; "
          f"first divergence (request: index, oracle gap) {gaps}")
    assert all(0 <= gap <= 1e-2 for _, gap in gaps.values()), gaps
    # Random-init weights give flat logits: which near-ties break which way
    # moves with any last-bit change of the arithmetic (5-6 of 8 identical
    # measured, every divergence at an oracle gap below 6e-4); the gap bound
    # above is the parity check, the count bounds how often ties occur.
    assert len(gaps) <= 3, gaps
    model.reset_all()


def test_fp16_artifact_graph_equals_eager(model):
    rng = np.random.default_rng(33)
    ids = rng.integers(0, 50257, 25).tolist()
    say("fp16 artifact: graph vs eager")
    model.reset_all()
    model.forward([0, 1], [ids, ids], return_logits=False, return_next=False)
    for tok in (ids[-1], 7, 50000):
        graph = logits_of(model.forward([0], [[tok]], return_next=True))
        eager = logits_of(model.forward([1], [[tok]], return_next=False))
        assert np.array_equal(graph, eager)
    model.reset_all()
