"""A greedy id outside the vocabulary (every logit non-finite: NaN never wins
the argmax, which then returns INT_MAX, reference llm/src/runtime.cu:59-66)
ends ti_llm_greedy_batch as the reference's loop ends it
(reference llm/src/runtime.cu:190-203): the id is written to the output, the
next forward rejects it as its input token (status INVALID, :160), the
lengths keep the forwards that ran, and the model stays usable (not
poisoned).  The artifact's weights are N(0, 300): finite in fp16, but the
activations overflow, so the logits are NaN from the prefill on."""
import pytest

pytestmark = pytest.mark.gpu

TINY = {"layers": 2, "heads": 2, "hidden": 128, "vocab": 300, "capacity": 64, "gelu": "gelu_new",
        "layer_norm_eps": 1e-5}
INT_MAX = 2**31 - 1


@pytest.fixture(scope="module")
def overflowing(tmp_path_factory):
    from tinyinfer_amd.artifact import write_synthetic
    return write_synthetic(tmp_path_factory.mktemp("tiny_nan"), TINY, seed=5, std=300.0)


def test_nonfinite_logits_end_greedy_as_invalid(overflowing):
    from tinyinfer_amd import LLM_LIB
    from tinyinfer_amd.runtime import NativeModel
    print("[case] greedy over NaN logits: INVALID, output kept, model usable", flush=True)
    with NativeModel(LLM_LIB, overflowing, max_batch=2, cache_slots=4, capacity=64) as m:
        # One token requested: no further forward, so the call succeeds and
        # returns the argmax of NaN logits as is.
        res = m.greedy([[1, 2, 3, 4]], 1, slots=[1])
        assert res["tokens"] == [[INT_MAX]]
        assert m.lengths()[1] == 4
        # More tokens: the first decode forward rejects the id.
        with pytest.raises(RuntimeError, match="status 1"):
            m.greedy([[1, 2, 3, 4], [5, 6]], 3, slots=[0, 2])
        lengths = m.lengths()
        assert lengths[0] == 4 and lengths[2] == 2, lengths  # the prefill ran, nothing after it
        # Not poisoned: the context still serves calls.
        m.reset(0)
        out = m.forward([0], [[7, 8, 9]], return_logits=True, return_next=True)
        assert m.lengths()[0] == 3
        assert len(out["logits"]) == TINY["vocab"] and len(out["next_tokens"]) == 1
