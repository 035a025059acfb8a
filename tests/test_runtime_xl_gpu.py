"""GPT-2 XL through libtinyinfer_llm.so (BASELINE configs[4] architecture:
hidden 1600, 25 heads x 64, MLP 6400, vocab 50257).

Against the CPU oracle (restating reference llm/src/runtime.cu), on a 2-layer
synthetic INT8 artifact with XL's shapes: K = 1600 and 6400 (25 and 100 chunks
of the packed GEMV/GEMM), N = 4800 / 1600 / 6400 / 50257, 25-head attention,
and the fused residual+LayerNorm finisher at 1600 columns.  Tolerances as the
small model: logits within atol 5e-2; greedy tokens identical, or diverging only
at near-ties (the oracle's own logit gap between the two picks at most 1e-2),
with the first divergence per request reported.  configs[4]'s own workload (64
requests, prompts U[128,512], KV capacity 640) runs here against the oracle.

On the full 48-layer artifact, where the oracle would take hours, the checks are
properties: a request's logits are bit-identical alone and inside the
64-request run, and the captured decode graph equals the eager path.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

NEW_TOKENS = 16


def say(*args):
    print("[case]", *args, flush=True)


@pytest.fixture(scope="module")
def artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import GPT2_XL, write_synthetic
    say("writing 2-layer GPT-2 XL-shaped synthetic artifact")
    return write_synthetic(tmp_path_factory.mktemp("gpt2xl2"), dict(GPT2_XL, layers=2), seed=7)


@pytest.fixture(scope="module")
def model(artifact):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    say("creating native XL-shaped model")
    with NativeModel(LLM_LIB, artifact, max_batch=8, cache_slots=9, capacity=512) as m:
        yield m


@pytest.fixture(scope="module")
def cpu_model(artifact):
    from tinyinfer_amd.artifact import load_tensors
    manifest, tensors = load_tensors(artifact)
    m = oracle.Gpt2(tensors, manifest["architecture"], slots=9, capacity=512)
    yield m
    m.close()


def logits_of(result):
    return np.frombuffer(result["logits"], dtype=np.float32).reshape(result["shape"]).copy()


def test_xl_logits_match_oracle(model, cpu_model):
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 50257, n).tolist() for n in (300, 37, 1, 130)]
    slots = [0, 1, 2, 3]
    say("xl logits vs oracle")
    model.reset_all()
    gpu = logits_of(model.forward(slots, prompts))
    for s in slots:
        cpu_model.reset(s)
    cpu, nxt = cpu_model.forward(slots, prompts)
    err = np.abs(gpu - cpu)
    print(f"prefill max |logit diff| {err.max():.3g}")
    assert err.max() <= 5e-2
    for _ in range(3):  # decode steps (captured graph path) on top of the prefill
        step = [[int(t)] for t in nxt]
        gpu2 = logits_of(model.forward(slots, step))
        cpu2, nxt = cpu_model.forward(slots, step)
        print(f"decode max |logit diff| {np.abs(gpu2 - cpu2).max():.3g}")
        assert np.abs(gpu2 - cpu2).max() <= 5e-2
    model.reset_all()


def first_divergence(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return i
    return None if len(a) == len(b) else min(len(a), len(b))


def test_xl_greedy_matches_oracle(model, cpu_model):
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, 50257, n).tolist() for n in (128, 200, 17, 64)]
    say("xl greedy vs oracle")
    model.reset_all()
    gpu = model.greedy(prompts, NEW_TOKENS)["tokens"]
    for s in range(len(prompts)):
        cpu_model.reset(s)
    cpu = cpu_model.greedy(list(range(len(prompts))), prompts, NEW_TOKENS)
    diverged = {b: i for b, i in ((b, first_divergence(g, c)) for b, (g, c) in enumerate(zip(gpu, cpu)))
                if i is not None}
    margins = {}
    for b, i in diverged.items():
        cpu_model.reset(8)
        lg, _ = cpu_model.forward([8], [prompts[b] + cpu[b][:i]])
        margins[b] = float(lg[0][cpu[b][i]] - lg[0][gpu[b][i]])
    print(f"xl greedy: {len(prompts) - len(diverged)}/{len(prompts)} identical over {NEW_TOKENS} tokens; "
          f"first divergence index {diverged}; oracle logit gap at divergence {margins}")
    assert all(0 <= m <= 1e-2 for m in margins.values()), margins
    model.reset_all()


@pytest.mark.parametrize("batch", [1, 20])
def test_xl_decode_batch_sizes_match_oracle(artifact, batch):
    """XL-shaped decode at 1 row (row-major activations) and at 20 rows (two
    16-row MFMA tiles over P32 fragment-packed activations): the residual GEMVs
    split K and the one-wave-per-row finisher sums the partials, adds bias and
    residual and writes the next LayerNorm.  Logits after a ragged prefill and
    two decode steps within atol 5e-2 of the oracle."""
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.artifact import load_tensors
    from tinyinfer_amd.runtime import NativeModel
    rng = np.random.default_rng(100 + batch)
    prompts = [rng.integers(0, 50257, int(n)).tolist() for n in rng.integers(1, 40, batch)]
    slots = list(range(batch))
    manifest, tensors = load_tensors(artifact)
    cpu = oracle.Gpt2(tensors, manifest["architecture"], slots=batch, capacity=64)
    try:
        say(f"xl decode, batch {batch}")
        with NativeModel(LLM_LIB, artifact, max_batch=batch, cache_slots=batch, capacity=64) as m:
            gpu = logits_of(m.forward(slots, prompts))
            ref, nxt = cpu.forward(slots, prompts)
            print(f"batch {batch} prefill max |logit diff| {np.abs(gpu - ref).max():.3g}")
            assert np.abs(gpu - ref).max() <= 5e-2
            for _ in range(2):
                step = [[int(t)] for t in nxt]
                gpu = logits_of(m.forward(slots, step))
                ref, nxt = cpu.forward(slots, step)
                print(f"batch {batch} decode max |logit diff| {np.abs(gpu - ref).max():.3g}")
                assert np.abs(gpu - ref).max() <= 5e-2
    finally:
        cpu.close()


# ---------------------------------------------------------------- configs[4] workload
# configs[4]'s 128 greedy tokens per request.
WORKLOAD_TOKENS = 128


def configs4_prompts():
    """64 requests, prompt lengths U[128,512] and ids U[0,50257) from seed 42
    (the bench's configs[4] workload)."""
    rng = np.random.default_rng(42)
    lens = rng.integers(128, 513, 64)
    return [rng.integers(0, 50257, int(n)).tolist() for n in lens]


HALVES = (list(range(0, 32)), list(range(32, 64)))  # max_batch slices, as the server batches


def test_xl_configs4_workload_vs_oracle(artifact):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.artifact import load_tensors
    from tinyinfer_amd.runtime import NativeModel
    prompts = configs4_prompts()
    say("configs[4] workload on the 2-layer XL-shaped artifact: GPU side")
    with NativeModel(LLM_LIB, artifact, max_batch=32, cache_slots=64, capacity=640) as m:
        gpu_prefill = np.concatenate([logits_of(m.forward(sl, [prompts[i] for i in sl])) for sl in HALVES])
        manifest, tensors = load_tensors(artifact)
        cpu = oracle.Gpt2(tensors, manifest["architecture"], slots=64, capacity=640)
        try:
            say("configs[4] workload: oracle prefill of 64 prompts")
            cpu_prefill, first = [], []
            for sl in HALVES:
                lg, nxt = cpu.forward(sl, [prompts[i] for i in sl])
                cpu_prefill.append(lg)
                first += [int(t) for t in nxt]
            cpu_prefill = np.concatenate(cpu_prefill)
            err = np.abs(gpu_prefill - cpu_prefill).max()
            print(f"configs[4] prefill of 64 requests: max |logit diff| {err:.3g}")
            assert err <= 5e-2
            # One decode step on both sides from the oracle's first token.
            gpu_step = np.concatenate([logits_of(m.forward(sl, [[first[i]] for i in sl])) for sl in HALVES])
            cpu_step, second = [], []
            for sl in HALVES:
                lg, nxt = cpu.forward(sl, [[first[i]] for i in sl])
                cpu_step.append(lg)
                second += [int(t) for t in nxt]
            err = np.abs(gpu_step - np.concatenate(cpu_step)).max()
            print(f"configs[4] first decode step of 64 requests: max |logit diff| {err:.3g}")
            assert err <= 5e-2
            say("configs[4] workload: GPU greedy")
            m.reset_all()
            gpu_tokens = []
            for sl in HALVES:
                gpu_tokens += m.greedy([prompts[i] for i in sl], WORKLOAD_TOKENS, slots=sl)["tokens"]
            say("configs[4] workload: oracle greedy continues")
            cpu_tokens = [[first[b], second[b]] for b in range(64)]
            gaps = {}

            def note(step, lg_by_request):
                for b, lg in lg_by_request:
                    if b in gaps:
                        continue
                    c, g = cpu_tokens[b][step], gpu_tokens[b][step]
                    if c != g:
                        gaps[b] = (step, float(lg[c] - lg[g]))

            note(0, zip(range(64), cpu_prefill))
            note(1, zip(range(64), np.concatenate(cpu_step)))
            for step in range(2, WORKLOAD_TOKENS):
                for sl in HALVES:
                    lg, nxt = cpu.forward(sl, [[cpu_tokens[i][-1]] for i in sl])
                    for i, t in zip(sl, nxt):
                        cpu_tokens[i].append(int(t))
                    note(step, zip(sl, lg))
        finally:
            cpu.close()
    print(f"configs[4] greedy, 64 requests x {WORKLOAD_TOKENS} tokens: {64 - len(gaps)}/64 identical; "
          f"first divergence (request: index, oracle gap) {gaps}")
    # Measured on MI355X: 53/64 requests identical over 128 tokens, every
    # divergence at an oracle gap <= 0.0015 (a near-tie; the kernels and the
    # oracle are deterministic, so the count is a property of the code, not of
    # the run).  Bounds: at most 12 diverging requests, gaps <= 5e-3.
    assert all(0 <= gap <= 5e-3 for _, gap in gaps.values()), gaps
    assert len(gaps) <= 12, gaps


def test_xl_configs4_concurrent_halves_equal_sequential(artifact):
    """configs[4]'s dynamic batch of 64 as two contexts of 32 decoding at the same
    time (one host thread each, as bench.py runs it) gives every request the
    tokens the sequential plan (one context, the halves one after the other)
    gives it: contexts share nothing and a request's sums do not depend on its
    batch."""
    import threading
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    prompts = configs4_prompts()
    new = 32
    say("configs[4] on the 2-layer XL-shaped artifact: sequential halves in one context")
    with NativeModel(LLM_LIB, artifact, max_batch=32, cache_slots=64, capacity=640) as m:
        seq = []
        for sl in HALVES:
            seq += m.greedy([prompts[i] for i in sl], new, slots=sl)["tokens"]
    say("configs[4]: the two halves at once, two contexts, two threads")
    with NativeModel(LLM_LIB, artifact, max_batch=32, cache_slots=32, capacity=640) as m0, \
            NativeModel(LLM_LIB, artifact, max_batch=32, cache_slots=32, capacity=640) as m1:
        out, errors = [None, None], []

        def work(i, model):
            try:
                out[i] = model.greedy([prompts[j] for j in HALVES[i]], new)["tokens"]
            except Exception as e:
                errors.append(e)
        threads = [threading.Thread(target=work, args=(i, mm)) for i, mm in enumerate((m0, m1))]
        for t in threads:
            t.start()
        for t in threads:
            t.join()
        assert not errors, errors
    assert out[0] + out[1] == seq


# ---------------------------------------------------------------- 48 layers: properties
@pytest.fixture(scope="module")
def xl48_artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import GPT2_XL, write_synthetic
    say("writing the 48-layer GPT-2 XL synthetic artifact (1.7 GB)")
    return write_synthetic(tmp_path_factory.mktemp("gpt2xl48"), GPT2_XL, seed=42)


def test_xl48_batch_invariance_and_graph_equals_eager(xl48_artifact):
    """Full GPT-2 XL, configs[4]'s 64 requests in two max_batch slices: requests
    alone give the same logits bits as inside the batched run, at prefill and at
    a decode step; the captured decode graph gives the eager path's bits."""
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    prompts = configs4_prompts()
    picks = (3, 40, 63)
    with NativeModel(LLM_LIB, xl48_artifact, max_batch=32, cache_slots=64, capacity=640) as m:
        say("xl48: batched prefill and graph decode step of 64 requests")
        pre, dec = {}, {}
        for sl in HALVES:
            lg = logits_of(m.forward(sl, [prompts[i] for i in sl]))
            for j, i in enumerate(sl):
                pre[i] = lg[j]
            step = logits_of(m.forward(sl, [[7] for _ in sl], return_next=True))  # graph path
            for j, i in enumerate(sl):
                dec[i] = step[j]
        say("xl48: the same requests alone")
        for i in picks:
            m.reset(i)
            alone = logits_of(m.forward([i], [prompts[i]]))[0]
            assert np.array_equal(alone, pre[i]), f"request {i}: prefill alone differs from the batched run"
            alone = logits_of(m.forward([i], [[7]], return_next=True))[0]
            assert np.array_equal(alone, dec[i]), f"request {i}: decode step alone differs from the batched run"
        say("xl48: graph vs eager decode")
        m.reset_all()
        m.forward([0, 1], [prompts[5], prompts[5]], return_logits=False, return_next=False)
        for tok in (11, 50000, 7):
            graph = logits_of(m.forward([0], [[tok]], return_next=True))
            eager = logits_of(m.forward([1], [[tok]], return_next=False))
            assert np.array_equal(graph, eager)
