"""GPU checks of libtinyinfer_llm.so through its C ABI (NativeModel mirror of
reference llm/runtime.py) on a seeded random-init GPT-2 small INT8 artifact
(BASELINE configs[0]).

* the reference's own model gate, reference llm/gpu_correctness.py:16-91 —
  batched == single, cached prefix == full, reset isolation, transactional
  rejection, scoring leaves public slots alone, masked NLL, mixed-length greedy
  == independent requests, GPU argmax == logits argmax, every trace counter > 0
  (cached tolerances atol 0.03 / rtol 0.005, reference llm/configs/evaluation.json);
* parity with the CPU oracle's GPT-2 (restating reference llm/src/runtime.cu):
  logits within atol 5e-2, greedy tokens identical at b=1 and b=32 (32-token
  prompts, 64 new tokens), the first divergence index reported otherwise;
* the captured decode graph gives bit-identical logits to the eager path.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

CACHED_ATOL, CACHED_RTOL = 0.03, 0.005
NEW_TOKENS = 64


def say(*args):
    print("[case]", *args, flush=True)


@pytest.fixture(scope="module")
def artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import GPT2_SMALL, write_synthetic
    say("writing GPT-2 small synthetic artifact")
    return write_synthetic(tmp_path_factory.mktemp("gpt2s"), GPT2_SMALL, seed=42)


@pytest.fixture(scope="module")
def model(artifact):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    say("creating native model")
    with NativeModel(LLM_LIB, artifact, max_batch=32, cache_slots=34, capacity=256) as m:
        yield m


@pytest.fixture(scope="module")
def cpu_model(artifact):
    from tinyinfer_amd.artifact import load_tensors
    manifest, tensors = load_tensors(artifact)
    m = oracle.Gpt2(tensors, manifest["architecture"], slots=34, capacity=256)
    yield m
    m.close()


def logits_of(result):
    return np.frombuffer(result["logits"], dtype=np.float32).reshape(result["shape"]).copy()


def token_ids(n, seed=42):
    return np.random.default_rng(seed).integers(0, 50257, n).tolist()


def test_reference_model_gate(model):
    ids = token_ids(64)
    prompts = [ids[0:33], ids[41:58]]
    say("model gate: independent vs batched")
    model.reset_all()
    independent = []
    for p in prompts:
        model.reset(0)
        r = model.forward([0], [p])
        lg = logits_of(r)
        assert np.all(np.isfinite(lg)) and r["next_tokens"] == lg.argmax(-1).tolist()
        independent.append(lg[0])
    full = np.stack(independent)
    model.reset_all()
    batched = logits_of(model.forward([0, 1], prompts))
    np.testing.assert_allclose(batched, full, atol=CACHED_ATOL, rtol=CACHED_RTOL)
    say("model gate: cached prefix")
    model.reset_all()
    model.forward([0, 1], [p[:3] for p in prompts], return_logits=False, return_next=False)
    cached = logits_of(model.forward([0, 1], [p[3:] for p in prompts]))
    np.testing.assert_allclose(cached, full, atol=CACHED_ATOL, rtol=CACHED_RTOL)
    say("model gate: reset isolation")
    model.reset(0)
    survivor = logits_of(model.forward([1], [[ids[59]]]))
    model.reset(2)
    expected = logits_of(model.forward([2], [prompts[1] + [ids[59]]]))
    np.testing.assert_allclose(survivor, expected, atol=CACHED_ATOL, rtol=CACHED_RTOL)
    before = model.lengths()
    for slots, rows in (([1, 1], [[3], [4]]), ([1], [[3] * model.options.capacity])):
        with pytest.raises(RuntimeError):
            model.forward(slots, rows, return_logits=False, return_next=False)
        assert model.lengths() == before
    say("model gate: scoring")
    score = model.score(ids[:33], [0] + [1] * 32, positions=True)
    assert model.lengths() == before and score["target_count"] == 32
    assert abs(sum(score["position_nll"]) - score["sum_nll"]) <= 1e-7 * max(1.0, score["sum_nll"])
    subset_mask = [0] + [int(i % 3 != 0) for i in range(1, 33)]
    subset = model.score(ids[:33], subset_mask, positions=True)
    want = sum(v for v, use in zip(score["position_nll"], subset_mask) if use)
    assert subset["target_count"] == sum(subset_mask) and model.lengths() == before
    assert abs(subset["sum_nll"] - want) <= 1e-7 * max(1.0, want)
    assert all(v == 0 for v, use in zip(subset["position_nll"], subset_mask) if not use)
    say("model gate: mixed greedy")
    model.reset_all()
    gen_prompts, requested = [prompts[0][:7], prompts[1][:5]], [3, 1]
    mixed = model.greedy(gen_prompts, requested, slots=[0, 1])
    assert mixed["output_lengths"] == requested and model.lengths()[:2] == [9, 5]
    for row, count, generated in zip(gen_prompts, requested, mixed["tokens"]):
        model.reset(2)
        assert model.greedy([row], count, slots=[2])["tokens"][0] == generated
    trace = model.trace()
    for key in ("embedding", "gemm_int8", "layernorm", "gelu", "attention", "residual", "kv_scatter_gather",
                "lm_head", "argmax", "nll"):
        assert trace[key] > 0, key
    model.reset_all()


def test_score_matches_oracle_nll(model, cpu_model):
    ids = token_ids(40, seed=7)
    say("score vs oracle")
    model.reset_all()
    score = model.score(ids, [0] + [1] * 39, positions=True)
    cpu_model.reset(0)
    lg = []
    for t in range(1, 40):
        cpu_model.reset(0)
        lg.append(cpu_model.forward([0], [ids[:t]])[0][0])
    lg = np.array(lg, np.float64)
    m = lg.max(1, keepdims=True)
    nll = (m[:, 0] + np.log(np.exp(lg - m).sum(1))) - lg[np.arange(39), ids[1:]]
    np.testing.assert_allclose(score["position_nll"][1:], nll, atol=5e-2)


def test_logits_match_oracle(model, cpu_model):
    ids = token_ids(100, seed=3)
    prompts = [ids[:32], ids[32:50], ids[50:51]]
    say("logits vs oracle")
    model.reset_all()
    gpu = logits_of(model.forward([0, 1, 2], prompts))
    for s in (0, 1, 2):
        cpu_model.reset(s)
    cpu, nxt = cpu_model.forward([0, 1, 2], prompts)
    err = np.abs(gpu - cpu)
    print(f"max |logit diff| {err.max():.3g}")
    assert err.max() <= 5e-2
    # one decode step on top of the prefill
    step = [[int(t)] for t in nxt]
    gpu2 = logits_of(model.forward([0, 1, 2], step))
    cpu2, _ = cpu_model.forward([0, 1, 2], step)
    assert np.abs(gpu2 - cpu2).max() <= 5e-2
    model.reset_all()


def test_decode_b17_and_one_row_score_match_oracle(model, cpu_model):
    """Decode of 17 requests (two 16-row MFMA tiles, the second mostly padding
    rows of the fragment-packed activations) and a two-token score (a one-row
    pass, whose ln_f output the head reads fragment-packed) against the oracle."""
    ids = token_ids(17 * 3 + 2, seed=13)
    prompts = [ids[3 * i:3 * i + 3] for i in range(17)]
    slots = list(range(17))
    say("decode b17 vs oracle")
    model.reset_all()
    model.forward(slots, prompts, return_logits=False, return_next=False)
    for s in slots:
        cpu_model.reset(s)
    _, nxt = cpu_model.forward(slots, prompts)
    step = [[int(t)] for t in nxt]
    res = model.forward(slots, step)
    gpu = logits_of(res)
    cpu, _ = cpu_model.forward(slots, step)
    print(f"b17 decode max |logit diff| {np.abs(gpu - cpu).max():.3g}")
    assert np.abs(gpu - cpu).max() <= 5e-2
    # the device's greedy pick (the head's per-workgroup partials) is the
    # lowest-index maximum of the logits it returned
    assert res["next_tokens"] == np.argmax(gpu, axis=1).tolist()
    say("two-token score vs oracle")
    pair = ids[-2:]
    sc = model.score(pair, [0, 1], positions=True)
    cpu_model.reset(0)
    lg = np.asarray(cpu_model.forward([0], [pair[:1]])[0][0], np.float64)
    m = lg.max()
    want = m + np.log(np.exp(lg - m).sum()) - lg[pair[1]]
    assert abs(sc["position_nll"][1] - want) <= 5e-2
    model.reset_all()


def test_long_prefill_matches_oracle(model, cpu_model):
    """16 requests of 128 tokens: a 2048-row prefill, where the linears run on
    the pre-dequantised fp16 weights (64 x 64 tiles) instead of the int8 panels."""
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, 50257, 128).tolist() for _ in range(16)]
    slots = list(range(16))
    say("2048-row prefill vs oracle")
    model.reset_all()
    gpu = logits_of(model.forward(slots, prompts))
    for s in slots:
        cpu_model.reset(s)
    cpu, nxt = cpu_model.forward(slots, prompts)
    print(f"2048-row prefill max |logit diff| {np.abs(gpu - cpu).max():.3g}")
    assert np.abs(gpu - cpu).max() <= 5e-2
    step = [[int(t)] for t in nxt]
    gpu2 = logits_of(model.forward(slots, step))
    cpu2, _ = cpu_model.forward(slots, step)
    assert np.abs(gpu2 - cpu2).max() <= 5e-2
    model.reset_all()


def test_decode_graph_equals_eager(model):
    ids = token_ids(20, seed=9)
    say("graph vs eager")
    model.reset_all()
    model.forward([0, 1], [ids, ids], return_logits=False, return_next=False)
    graph = model.forward([0], [[ids[-1]]], return_logits=True, return_next=True)  # captured path
    eager = model.forward([1], [[ids[-1]]], return_logits=True, return_next=False)  # eager path
    assert np.array_equal(logits_of(graph), logits_of(eager))
    for _ in range(3):  # replays with advancing positions keep agreeing
        g = model.forward([0], [[7]], return_logits=True, return_next=True)
        e = model.forward([1], [[7]], return_logits=True, return_next=False)
        assert np.array_equal(logits_of(g), logits_of(e))
    model.reset_all()


@pytest.mark.parametrize("others", [1, 4, 15, 20, 31])
def test_prefill_and_decode_are_batch_invariant(model, others):
    """A request's logits do not depend on the batch it runs in: its prompt
    prefilled alone or beside others of other lengths (rows of the prefill GEMMs
    and attention summed in one order whatever the batch), then decode steps of
    1 to 32 rows (the 32-row GEMVs and LM head sum K in the 16-row kernels'
    order).  The epoll server batches requests as they arrive and its greedy
    output must equal direct greedy decoding."""
    ids = token_ids(24, seed=11)
    rows = [token_ids(5 + 3 * i, seed=100 + i) for i in range(others)]
    say("batch invariance", others)
    model.reset_all()
    alone = logits_of(model.forward([0], [ids]))[0]
    batched = logits_of(model.forward(list(range(1, others + 2)), [ids] + rows))[0]
    assert np.array_equal(alone, batched)
    for tok in (ids[-1], 7, 50000):
        alone = logits_of(model.forward([0], [[tok]]))[0]
        batched = logits_of(model.forward(list(range(1, others + 2)), [[tok]] + [[3]] * others))[0]
        assert np.array_equal(alone, batched)
    model.reset_all()


def test_long_prefill_batch_invariant(model):
    """32 prompts of 150..255 ids prefill with two 16-query blocks per attention
    wave (>= 512 workgroups of 128 queries), a prompt alone with one: the same
    logits bits (a query's attention sums do not depend on the blocking)."""
    rng = np.random.default_rng(12)
    rows = [rng.integers(0, 50257, int(n)).tolist() for n in rng.integers(150, 256, 32)]
    say("long prefill batch invariance")
    model.reset_all()
    batched = logits_of(model.forward(list(range(32)), rows))
    for i in (0, 17, 31):
        model.reset(33)
        alone = logits_of(model.forward([33], [rows[i]]))[0]
        assert np.array_equal(alone, batched[i]), f"request {i}"
    model.reset_all()


def first_divergence(a, b):
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y:
            return i
    return None if len(a) == len(b) else min(len(a), len(b))


@pytest.mark.parametrize("batch", [17, 31])
def test_greedy_runs_and_lanes_match_alone(model, batch):
    """ti_llm_greedy_batch decodes in runs (each run advances every unfinished
    request by the fewest tokens any still needs) and splits a run of more than
    16 requests into two lanes: with ragged prompt lengths and token counts the
    active set shrinks run by run and the lanes split unevenly (9 + 8, 16 + 15,
    then smaller), yet every request's tokens, output lengths and timings
    match the request decoded alone."""
    rng = np.random.default_rng(batch)
    prompts = [rng.integers(0, 50257, int(n)).tolist() for n in rng.integers(1, 40, batch)]
    counts = [int(c) for c in rng.integers(1, 48, batch)]
    counts[0], counts[-1] = 47, 1
    say("greedy runs and lanes, batch", batch)
    model.reset_all()
    res = model.greedy(prompts, counts)
    assert res["output_lengths"] == counts
    assert all(0 < f <= t for f, t in zip(res["ttft_ms"], res["total_ms"]))
    for i in (0, 1, batch // 2, batch - 1):
        model.reset_all()
        alone = model.greedy([prompts[i]], counts[i], slots=[33])
        assert alone["tokens"][0] == res["tokens"][i], f"request {i}"
    model.reset_all()


@pytest.mark.parametrize("batch", [1, 32])
def test_greedy_tokens_match_oracle(model, cpu_model, batch):
    """32 seeded uniform prompt ids per request, 64 greedy tokens."""
    rng = np.random.default_rng(42)
    prompts = [rng.integers(0, 50257, 32).tolist() for _ in range(batch)]
    say("greedy vs oracle, batch", batch)
    model.reset_all()
    gpu = model.greedy(prompts, NEW_TOKENS)["tokens"]
    for s in range(batch):
        cpu_model.reset(s)
    cpu = cpu_model.greedy(list(range(batch)), prompts, NEW_TOKENS)
    report = {b: first_divergence(g, c) for b, (g, c) in enumerate(zip(gpu, cpu))}
    diverged = {b: i for b, i in report.items() if i is not None}
    # At a divergence both sides agree on every earlier token; the oracle's logits at
    # that step show whether the two picks are a near-tie (gap within the 5e-2 logits
    # tolerance) or a real disagreement.
    margins = {}
    for b, i in diverged.items():
        cpu_model.reset(33)
        lg, _ = cpu_model.forward([33], [prompts[b] + cpu[b][:i]])
        margins[b] = float(lg[0][cpu[b][i]] - lg[0][gpu[b][i]])
    print(f"greedy batch {batch}: {batch - len(diverged)}/{batch} identical over {NEW_TOKENS} tokens; "
          f"first divergence index {diverged}; oracle logit gap at divergence {margins}")
    # A divergence is accepted only at a near-tie: the oracle's own gap between
    # the two picks at most 1e-2 (about twice the measured GPU-vs-oracle logit
    # error, 0.004), and at most a quarter of the requests may diverge at all.
    assert all(0 <= m <= 1e-2 for m in margins.values()), margins
    assert len(diverged) <= batch // 4, diverged
    model.reset_all()
