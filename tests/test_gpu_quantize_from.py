"""q_llama_quantize_from (llama.c:490-511) on the GPU against the compiled
reference: an fp32 LlamaModel quantized per column on the device gives the
reference's int8 model (digest of every code and scale) and its decode steps
give the reference's logits bit for bit (fixtures of tests/golden/gen_golden.c
qfrom: selftest [21]'s model shape, and a model with gains and biases)."""
import numpy as np
import pytest

import oracle_lib as O
import qlib
from conftest import golden, golden_json

pytestmark = pytest.mark.gpu

CASES = ["selftest21", "biased"]


@pytest.fixture(scope="module")
def Q():
    return qlib.load()


@pytest.mark.parametrize("name", CASES)
def test_quantize_from_matches_reference(Q, name):
    meta = golden_json(f"qfrom_{name}")
    cfg = meta["cfg"]
    tensors = O.qfrom_tensors(cfg, meta["gain_sigma"], meta["bias_sigma"], seed=meta["seed"])
    assert O.tensors_hash(tensors) == int(meta["fp32_hash"], 16)
    want = golden(f"qfrom_{name}_logits")
    m = Q.Model.quantize_from(cfg, meta["rope_base"], 1e-5, tensors)
    try:
        assert m.hash() == int(meta["model_hash"], 16)
        for i, t in enumerate(meta["tokens"]):
            got = m.step(t)
            assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), f"{name}: step {i}"
    finally:
        m.close()
