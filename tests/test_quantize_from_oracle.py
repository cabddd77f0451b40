"""The oracle's restatement of q_llama_quantize_from (llama.c:490-511) against
the compiled reference's fixtures (tests/golden/gen_golden.c qfrom): the same
int8 model (digest of every code and scale) and the same logits at every step."""
import numpy as np
import pytest

import oracle_lib as O
from conftest import golden, golden_json


@pytest.mark.parametrize("name", ["selftest21", "biased"])
def test_oracle_quantize_from_matches_reference(name):
    meta = golden_json(f"qfrom_{name}")
    cfg = meta["cfg"]
    tensors = O.qfrom_tensors(cfg, meta["gain_sigma"], meta["bias_sigma"], seed=meta["seed"])
    assert O.tensors_hash(tensors) == int(meta["fp32_hash"], 16)
    want = golden(f"qfrom_{name}_logits")
    m = O.Model.quantize_from(cfg, meta["rope_base"], 1e-5, tensors)
    try:
        assert m.hash() == int(meta["model_hash"], 16)
        for i, t in enumerate(meta["tokens"]):
            got = m.step(t)
            assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), f"{name}: step {i}"
        # the greedy continuation recorded in the fixture is the argmax of each step
        n = meta["n_prompt"]
        for i in range(n - 1, len(meta["tokens"]) - 1):
            assert int(np.argmax(want[i])) == meta["tokens"][i + 1]
    finally:
        m.close()


def test_oracle_quantize_from_zero_column_scale():
    """quant.c:14-16: an all-zero output column gets scale 1 and zero codes."""
    meta = golden_json("qfrom_biased")
    cfg = meta["cfg"]
    tensors = O.qfrom_tensors(cfg, meta["gain_sigma"], meta["bias_sigma"], seed=meta["seed"])
    m = O.Model.quantize_from(cfg, meta["rope_base"], 1e-5, tensors)
    try:
        lh = m.m.lm_head
        scale = np.ctypeslib.as_array(lh.scale, shape=(lh.cols,))
        codes = np.ctypeslib.as_array(lh.q, shape=(lh.rows, lh.cols))
        assert scale[5] == np.float32(1.0) and not codes[:, 5].any()
        assert (scale[np.arange(lh.cols) != 5] != 1.0).all()
    finally:
        m.close()
