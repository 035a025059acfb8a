"""Pins the CPU oracle (oracle/oracle.cpp) before it is trusted as the checker.

Each oracle function is checked against (a) the reference's golden vectors and
known answers (tests/golden/), (b) the reference's own CPU code compiled from
/root/reference (oracle/_ref, through the committed fixtures), and (c) what the
mathematics fixes — closed forms, invariants and independent float64 numpy
formulations — chosen so a dropped term, wrong sign/index or transposed operand
fails at least one check.
"""
import math

import numpy as np
import pytest

import oracle
from tests.conftest import GOLDEN


def f16(x):
    return np.asarray(x, np.float16).view(np.uint16)


def h(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


# ---------------------------------------------------------------- fp16 conversions
def test_f16_to_f32_all_patterns_match_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(1)
    vals = [rng.standard_normal(200000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 300, 3e4)]
    # Exact midpoints between consecutive halves (ties), subnormal ties and the overflow edge.
    halves = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 65536, 2**-24, 2**-25, 1.5 * 2**-25, 2**-26, 0, -0.0],
                    np.float32)
    x = np.concatenate(vals + [mids, -mids, edge, -edge])
    got = oracle.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


# ---------------------------------------------------------------- INT8 codec
def test_quantize_known_answers(golden):
    case = golden["quantize_output_axis"]
    q, s = oracle.quantize(f16(case["rows"]))
    assert s.tolist() == case["scales"] and q.tolist() == case["q"]
    assert h(oracle.dequantize(q, s)).tolist() == case["dequant"]
    ties = golden["quantize_ties_to_even"]
    q, s = oracle.quantize(f16(ties["rows"]))
    assert s.tolist() == ties["scales"] and q.tolist() == ties["q"]


def test_dequant_round_trip_is_fp16_and_close(golden):
    case = golden["dequant_round_trip"]
    w = f16(case["rows"])
    q, s = oracle.quantize(w)
    back = h(oracle.dequantize(q, s))
    assert np.abs(back - h(w)).max() < case["max_abs_error"]


@pytest.mark.parametrize("key", ["all_half", "fixed0", "fixed1", "fixed2", "fixed3", "random"])
def test_quantize_matches_reference_codec_bytes(key):
    v = np.load(GOLDEN / "codec_vectors.npz")
    q, s = oracle.quantize(v[key + "_in"])
    assert np.array_equal(q, v[key + "_q"])
    assert np.array_equal(s.view(np.uint32), v[key + "_s"].view(np.uint32))


def test_dequantize_matches_reference_codec_bytes():
    v = np.load(GOLDEN / "codec_vectors.npz")
    assert np.array_equal(oracle.dequantize(v["deq_q"], v["deq_s"]), v["deq_out"])


def test_quantize_closed_form_scale_and_clamp():
    rng = np.random.default_rng(2)
    w = f16(rng.standard_normal((33, 17)) * 0.05)
    q, s = oracle.quantize(w)
    wf = h(w)
    mx = np.abs(wf).max(axis=0)
    assert np.array_equal(s, (mx / 127.0).astype(np.float32))
    assert q.min() >= -127 and q.max() <= 127
    # the column maximum maps to exactly +-127
    idx = np.abs(wf).argmax(axis=0)
    assert np.all(np.abs(q[idx, np.arange(17)]) == 127)


# ---------------------------------------------------------------- linear
def _deq(q, s):
    return h(oracle.dequantize(q, s))


def test_linear_identity_selects_weight_rows_exactly():
    rng = np.random.default_rng(3)
    w = f16(rng.standard_normal((24, 40)) * 0.1)
    q, s = oracle.quantize(w)
    bias = f16(rng.standard_normal(40) * 0.1)
    a = f16(np.eye(24))
    y = oracle.linear(a, q=q, scales=s, bias_bits=bias)
    want = (_deq(q, s) + h(bias)[None, :]).astype(np.float32).astype(np.float16).view(np.uint16)
    assert np.array_equal(y, want)


def test_linear_matches_float64_product_and_orientation():
    rng = np.random.default_rng(4)
    m, k, n = 5, 96, 72
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    q[:, 3] = 0  # zero channel: output is the bias
    y = oracle.linear(a, q=q, scales=s, bias_bits=bias, out_dtype="f32")
    want = h(a) @ _deq(q, s) + h(bias)
    assert np.allclose(y, want, rtol=1e-5, atol=1e-5)
    assert np.array_equal(y[:, 3], h(bias)[3].repeat(m).astype(np.float32))
    # a transposed weight would not agree
    wrong = h(a) @ _deq(q, s)[::-1]
    assert not np.allclose(y, wrong + h(bias), rtol=1e-3, atol=1e-3)
    # fp16 weights path equals the int8 path on the dequantized weights
    y16 = oracle.linear(a, w_bits=oracle.dequantize(q, s), bias_bits=bias, out_dtype="f32")
    assert np.array_equal(y16, y)


def test_linear_gelu_epilogue_closed_form():
    rng = np.random.default_rng(5)
    a = f16(rng.standard_normal((3, 64)))
    w = f16(rng.standard_normal((64, 50)) * 0.2)
    bias = f16(rng.standard_normal(50) * 0.1)
    q, s = oracle.quantize(w)
    pre = h(oracle.linear(a, q=q, scales=s, bias_bits=bias))  # fp16-rounded biased values
    y = h(oracle.linear(a, q=q, scales=s, bias_bits=bias, gelu=True))
    want = 0.5 * pre * (1 + np.tanh(math.sqrt(2 / math.pi) * (pre + 0.044715 * pre**3)))
    assert np.allclose(y, want, rtol=2e-3, atol=2e-3)
    assert oracle.linear(f16(np.zeros((1, 64))), q=q, scales=s, gelu=True).max() == 0


@pytest.mark.parametrize("shape", [(1, 1, 1), (7, 13, 5), (33, 65, 70)])
def test_matmul_blocked_matches_reference_cpu(shape):
    m, n, k = shape
    v = np.load(GOLDEN / "cpu_kernel_vectors.npz")
    a, b, y = v[f"mm{m}_{n}_{k}_a"], v[f"mm{m}_{n}_{k}_b"], v[f"mm{m}_{n}_{k}_y"]
    got = oracle.matmul_blocked(a, b)
    assert np.allclose(got, y, atol=1e-5 * k + 1e-5)
    assert np.allclose(got, a.astype(np.float64) @ b, atol=1e-5 * k + 1e-5)


# ---------------------------------------------------------------- LayerNorm / Softmax fp32
@pytest.mark.parametrize("cols", [2, 64, 768, 1024, 4099])
def test_layernorm_f32_matches_reference(cols):
    v = np.load(GOLDEN / "cpu_kernel_vectors.npz")
    x, g, b, y = (v[f"ln{cols}_{s}"] for s in "xgby")
    assert np.allclose(oracle.layernorm_f32_fused(x, g, b), y, atol=1e-6, rtol=1e-6)
    exact = oracle.layernorm_f32_exact(x, g, b)
    assert np.allclose(exact, y, atol=1e-4)  # reference test tolerance, test_cpu.cpp:67
    xd = x.astype(np.float64)
    mu, var = xd.mean(1, keepdims=True), xd.var(1, keepdims=True)
    assert np.allclose(exact, (xd - mu) / np.sqrt(var + 1e-5) * g + b, atol=1e-6)


@pytest.mark.parametrize("cols", [1, 31, 128, 1000, 4097])
def test_softmax_f32_matches_reference(cols):
    v = np.load(GOLDEN / "cpu_kernel_vectors.npz")
    x, y = v[f"sm{cols}_x"], v[f"sm{cols}_y"]
    assert np.allclose(oracle.softmax_f32_fused(x), y, atol=1e-7)
    exact = oracle.softmax_f32_exact(x)
    assert np.allclose(exact, y, atol=1e-6)  # reference test tolerance, test_cpu.cpp:42
    assert np.allclose(exact.sum(1), 1, atol=1e-5)


def test_rowops_special_rows():
    x = np.full((1, 256), 3.25, np.float32)
    g, b = np.full(256, 2, np.float32), np.full(256, 0.5, np.float32)
    assert np.allclose(oracle.layernorm_f32_exact(x, g, b), 0.5, atol=1e-6)
    rng = np.random.default_rng(6)
    big = rng.uniform(1e4 - 1, 1e4 + 1, (3, 1024)).astype(np.float32)
    ones, zeros = np.ones(1024, np.float32), np.zeros(1024, np.float32)
    ref = oracle.layernorm_f32_exact(big, ones, zeros)
    assert np.allclose(oracle.layernorm_f32_fused(big, ones, zeros), ref, atol=5e-3)
    masked = rng.standard_normal((2, 40)).astype(np.float32)
    masked[:, ::3] = -np.inf
    y = oracle.softmax_f32_exact(masked)
    assert np.all(y[:, ::3] == 0) and np.allclose(y.sum(1), 1, atol=1e-6)


# ---------------------------------------------------------------- fp16 row ops
@pytest.mark.parametrize("cols", [1, 7, 257, 768, 3072])
def test_fp16_rowops_closed_forms(cols):
    rng = np.random.default_rng(cols)
    x = f16(rng.standard_normal((3, cols)))
    g, b = f16(rng.standard_normal(cols)), f16(rng.standard_normal(cols))
    xd = h(x)
    mu, var = xd.mean(1, keepdims=True), xd.var(1, keepdims=True)
    ln = (xd - mu) / np.sqrt(var + 1e-5) * h(g) + h(b)
    assert np.allclose(h(oracle.layernorm_f16(x, g, b)), ln, rtol=2e-3, atol=2e-3)
    e = np.exp(xd - xd.max(1, keepdims=True))
    assert np.allclose(h(oracle.softmax_f16(x)), e / e.sum(1, keepdims=True), rtol=2e-3, atol=1e-4)
    gl = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd**3)))
    assert np.allclose(h(oracle.gelu_f16(x)), gl, rtol=2e-3, atol=1e-4)


def test_fp16_layernorm_constant_row_gives_beta():
    x = f16(np.full((2, 96), 1.5))
    g, b = f16(np.full(96, 2.0)), f16(np.linspace(-1, 1, 96))
    assert np.array_equal(oracle.layernorm_f16(x, g, b), np.tile(b, (2, 1)))


# ---------------------------------------------------------------- attention
def _attention_f64(q, k, v, ql, kl, off, causal):
    qd, kd, vd = h(q), h(k), h(v)
    bsz, nh, nq, d = qd.shape
    out = np.zeros_like(qd)
    for b in range(bsz):
        for i in range(min(nq, ql[b])):
            n = min(kl[b], off[b] + i + 1) if causal else kl[b]
            if n <= 0:
                continue
            s = np.einsum("hd,hkd->hk", qd[b, :, i], kd[b, :, :n]) / math.sqrt(d)
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            out[b, :, i] = np.einsum("hk,hkd->hd", p, vd[b, :, :n])
    return out


@pytest.mark.parametrize("d", [64, 128])
def test_attention_reference_cases_against_float64(golden, d):
    rng = np.random.default_rng(7 + d)
    for nq, nk, ql, kl, off, causal in golden["attention_cases"]["cases"]:
        q = f16(rng.standard_normal((2, 2, nq, d)) * 0.5)
        k = f16(rng.standard_normal((2, 2, nk, d)) * 0.5)
        v = f16(rng.standard_normal((2, 2, nk, d)))
        got = h(oracle.attention_f16(q, k, v, ql, kl, off, causal))
        want = _attention_f64(q, k, v, ql, kl, off, causal)
        assert np.allclose(got, want, rtol=2e-3, atol=2e-3)
        # rows with no visible key are exactly zero
        for b in range(2):
            for i in range(nq):
                visible = min(kl[b], off[b] + i + 1) if causal else kl[b]
                if i >= ql[b] or visible <= 0:
                    assert np.all(got[b, :, i] == 0)


def test_attention_invariants():
    rng = np.random.default_rng(8)
    k = f16(rng.standard_normal((1, 1, 9, 64)))
    v = f16(rng.standard_normal((1, 1, 9, 64)))
    q = f16(rng.standard_normal((1, 1, 1, 64)))
    one = oracle.attention_f16(q, k, v, [1], [9], [0], True)  # causal, offset 0: key 0 only
    assert np.array_equal(one[0, 0, 0], v[0, 0, 0])
    zero_q = f16(np.zeros((1, 1, 1, 64)))
    mean = h(oracle.attention_f16(zero_q, k, v, [1], [9], [0], False))
    assert np.allclose(mean[0, 0, 0], h(v)[0, 0].mean(0), atol=1e-3)


# ---------------------------------------------------------------- GPT-2
TINY = {"layers": 2, "heads": 2, "hidden": 128, "vocab": 300, "capacity": 64, "gelu": "gelu_new",
        "layer_norm_eps": 1e-5}


@pytest.fixture(scope="module")
def tiny_artifact(tmp_path_factory):
    from tinyinfer_amd.artifact import write_synthetic
    return write_synthetic(tmp_path_factory.mktemp("tiny"), TINY, seed=11)


@pytest.fixture(scope="module")
def tiny_tensors(tiny_artifact):
    from tinyinfer_amd.artifact import load_tensors
    return load_tensors(tiny_artifact)[1]


@pytest.fixture(scope="module")
def tiny_f16_tensors(tmp_path_factory):
    from tinyinfer_amd.artifact import load_tensors, write_synthetic
    return load_tensors(write_synthetic(tmp_path_factory.mktemp("tiny16"), TINY, seed=11, precision="fp16"))[1]


def test_gpt2_self_consistency(tiny_tensors):
    m = oracle.Gpt2(tiny_tensors, TINY, slots=4, capacity=64)
    rng = np.random.default_rng(9)
    p0, p1 = rng.integers(0, 300, 17).tolist(), rng.integers(0, 300, 9).tolist()
    single = []
    for p in (p0, p1):
        m.reset(0)
        single.append(m.forward([0], [p])[0][0])
    m.reset(0)
    batched, nxt = m.forward([0, 1], [p0, p1])
    assert np.array_equal(batched, np.stack(single))
    assert nxt.tolist() == batched.argmax(1).tolist()
    for s in range(4):
        m.reset(s)
    m.forward([0, 1], [p0[:3], p1[:3]], logits=False)
    cached, _ = m.forward([0, 1], [p0[3:], p1[3:]])
    assert np.array_equal(cached, batched)
    assert [m.length(0), m.length(1)] == [17, 9]


def test_gpt2_mixed_greedy_lengths(tiny_tensors, golden):
    case = golden["mixed_greedy_lengths"]
    m = oracle.Gpt2(tiny_tensors, TINY, slots=4, capacity=64)
    rng = np.random.default_rng(10)
    prompts = [rng.integers(0, 300, n).tolist() for n in case["prompt_lengths"]]
    out = m.greedy([0, 1], prompts, case["requested"])
    assert [len(o) for o in out] == case["requested"]
    assert [m.length(0), m.length(1)] == case["lengths_after"]
    for prompt, n, gen in zip(prompts, case["requested"], out):
        m.reset(2)
        assert m.greedy([2], [prompt], n)[0] == gen


@pytest.mark.parametrize("precision", ["int8", "fp16"])
def test_gpt2_matches_independent_transformers_model(precision, request):
    """Cross-check against HF transformers' GPT-2 (float32, CPU) loaded with the same
    weights (dequantized INT8, or the fp16 linears of a float16 artifact as
    stored): an independent implementation of the architecture."""
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    cfg = tr.GPT2Config(vocab_size=300, n_positions=64, n_embd=128, n_layer=2, n_head=2,
                        activation_function="gelu_new", layer_norm_epsilon=1e-5,
                        resid_pdrop=0, embd_pdrop=0, attn_pdrop=0, tie_word_embeddings=False)
    model = tr.GPT2LMHeadModel(cfg).eval()
    t = tiny_tensors = request.getfixturevalue("tiny_tensors" if precision == "int8" else "tiny_f16_tensors")
    f = lambda bits: torch.tensor(h(bits), dtype=torch.float32)
    if precision == "int8":
        deq = lambda name: torch.tensor(_deq(t[name], t[name + ".scales"]), dtype=torch.float32)
    else:
        assert t["lm_head.weight"].dtype == np.uint16 and "lm_head.weight.scales" not in t
        deq = lambda name: f(t[name])
    sd = {"transformer.wte.weight": f(t["transformer.wte.weight"]),
          "transformer.wpe.weight": f(t["transformer.wpe.weight"]),
          "transformer.ln_f.weight": f(t["transformer.ln_f.weight"]),
          "transformer.ln_f.bias": f(t["transformer.ln_f.bias"]),
          "lm_head.weight": deq("lm_head.weight").T.contiguous()}
    for l in range(2):
        p = f"transformer.h.{l}."
        for ln in ("ln_1", "ln_2"):
            sd[p + ln + ".weight"], sd[p + ln + ".bias"] = f(t[p + ln + ".weight"]), f(t[p + ln + ".bias"])
        for lin in ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj"):
            sd[p + lin + ".weight"] = deq(p + lin + ".weight")
            sd[p + lin + ".bias"] = f(t[p + lin + ".bias"])
    missing, _ = model.load_state_dict(sd, strict=False)
    assert not [k for k in missing if not k.endswith(".attn.bias") and "masked_bias" not in k]
    rng = np.random.default_rng(12)
    ids = rng.integers(0, 300, 20).tolist()
    m = oracle.Gpt2(tiny_tensors, TINY, slots=1, capacity=64)
    ours, _ = m.forward([0], [ids])
    with torch.no_grad():
        theirs = model(torch.tensor([ids])).logits[0, -1].numpy()
    assert np.allclose(ours[0], theirs, atol=5e-3, rtol=1e-2)
