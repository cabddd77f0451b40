"""The oracle's fp32 (LLMA) decode path (llama.c:296-362, matrix.c:178-190) and
the tests' LLMA writer, pinned against fixtures the compiled reference wrote
(gen_golden e2e_f32) and against the reference's own loader.  CPU only."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O
from conftest import ROOT, golden, golden_json

REF_GEN = os.path.join(ROOT, "oracle", "_ref", "gen_golden")


def test_matmul_row_closed_forms():
    rng = np.random.default_rng(3)
    a = rng.standard_normal(37).astype(np.float32)
    W = rng.standard_normal((37, 11)).astype(np.float32)
    c = O.matmul_row(a, W)
    # k-order float sum of rounded products, written out
    ref = np.zeros(11, np.float32)
    for k in range(37):
        ref = (ref + (a[k] * W[k]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(c.view(np.uint32), ref.view(np.uint32))
    # identity rows select, zero input gives +0
    E = np.eye(5, dtype=np.float32)
    assert np.array_equal(O.matmul_row(np.arange(5, dtype=np.float32), E), np.arange(5, dtype=np.float32))
    assert not np.signbit(O.matmul_row(np.zeros(4, np.float32), -np.ones((4, 3), np.float32))).any()


@pytest.mark.parametrize("name", ["tiny", "mid"])
def test_f32_decode_matches_reference(name):
    meta = golden_json(f"e2e_f32_{name}")
    m = O.FModel(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    try:
        assert m.hash() == int(meta["model_hash"], 16)
        hashes = [int(h, 16) for h in meta["logit_hashes"]]
        P = len(meta["prompt"])
        for i, t in enumerate(meta["prompt"]):
            lg = m.step(t)
            assert O.hash_f32(lg) == hashes[i], i
        assert np.array_equal(lg.view(np.uint32), golden(f"e2e_f32_{name}_logits_prompt_last").view(np.uint32))
        for s, t in enumerate(meta["gen"]):
            assert int(np.argmax(lg)) == t
            lg = m.step(t)
            assert O.hash_f32(lg) == hashes[P + s], P + s
        assert np.array_equal(lg.view(np.uint32), golden(f"e2e_f32_{name}_logits_final").view(np.uint32))
    finally:
        m.close()


@pytest.mark.skipif(not os.path.exists(REF_GEN), reason="reference objects not built (no /root/reference)")
def test_llma_writer_round_trips_through_reference_loader(tmp_path):
    meta = golden_json("e2e_f32_tiny")
    m = O.FModel(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        path = tmp_path / "tiny.llma"
        m.write_llma(str(path))
        out = subprocess.run([REF_GEN, str(tmp_path), "llmahash", str(path)], capture_output=True, text=True,
                             check=True)
        assert int(out.stdout.strip(), 16) == m.hash()
    finally:
        m.close()


@pytest.mark.parametrize("name", ["tiny", "mid"])
def test_reference_forward_rows_are_its_decode_steps(name):
    """The fixtures record the reference's batched forward (llama.c:167-186) over
    the prompt: each row's digest equals that of its decode step, which is what
    lets the GPU's llama_model_forward run decode steps."""
    meta = golden_json(f"e2e_f32_{name}")
    P = len(meta["prompt"])
    assert meta["forward_hashes"] == meta["logit_hashes"][:P]
