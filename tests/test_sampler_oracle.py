"""The oracle's sampler (sampler.c:24-143) and the LLMQ writer the tests use,
pinned against fixtures written by the compiled reference (gen_golden sample)
and against the reference's own loader.  CPU only."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as O
from conftest import ROOT, golden_json

S = golden_json("sample")
TINY = [32000, 288, 6, 6, 2, 48, 768, 256]


def test_rng_uniform_matches_reference():
    for seed, *bits in S["uniform"]:
        st = O.rng_create(seed)
        for b in bits:
            u, st = O.rng_uniform(st)
            assert np.float32(u).view(np.uint32) == b


@pytest.mark.parametrize("ci", range(len(S["sample_cases"])))
def test_sample_token_matches_reference(ci):
    c = S["sample_cases"][ci]
    row = O.sample_row(c["V"], c["tid"], c["sigma"], c["kind"])
    st = O.rng_create(c["seed"])
    toks = []
    for _ in range(8):
        t, st = O.sample_token(row, c["t"], c["k"], c["p"], st)
        toks.append(t)
    assert toks == c["tokens"]
    assert st == int(c["state"], 16)


def test_sampler_fixtures_exercise_ties():
    # the quarter-rounded rows hold many equal probabilities inside the kept set,
    # so the fixtures decide the order of ties
    row = O.sample_row(32000, 2, 1.0, 1)
    top = np.sort(row)[::-1][:40]
    assert len(np.unique(top)) < 10


def test_top_k_one_is_argmax():
    # selftest.c:325-333: top_k = 1 returns the argmax whatever the draw
    for tid in range(3):
        row = O.sample_row(5000, 20 + tid, 1.0, 1)
        st = O.rng_create(123)
        for _ in range(4):
            t, st = O.sample_token(row, 1.0, 1, 1.0, st)
            assert t == O.lib().or_argmax(O.fptr(row), row.size)


def test_same_seed_same_stream():
    # selftest.c:335-345: two generators from one seed draw the same tokens
    row = O.sample_row(3000, 9, 1.0, 0)
    a = b = O.rng_create(7)
    for _ in range(16):
        ta, a = O.sample_token(row, 0.9, 40, 0.95, a)
        tb, b = O.sample_token(row, 0.9, 40, 0.95, b)
        assert ta == tb and a == b


def test_greedy_leaves_rng_untouched():
    row = O.sample_row(3000, 10, 1.0, 0)
    st = O.rng_create(99)
    t, st2 = O.sample_token(row, 0.0, 40, 0.95, st)
    assert st2 == st and t == int(np.argmax(row))


def test_cli_loop_oracle_matches_reference():
    """The `llama` command's sampled loop (main.c:658-669) on the tiny model."""
    cli = S["cli"]
    m = O.Model(TINY, 10000.0, seed=cli["seed"])
    try:
        st = O.rng_create(1234)
        for line in cli["lines"]:
            m.reset(0)
            for t in line["prompt"]:
                logits = m.step(t)
            gen = []
            for _ in range(cli["n_new"]):
                t, st = O.sample_token(logits, 0.8, 40, 0.95, st)
                gen.append(t)
                logits = m.step(t)
            assert gen == line["gen"]
    finally:
        m.close()


REF_GEN = os.path.join(ROOT, "oracle", "_ref", "gen_golden")


@pytest.mark.skipif(not os.path.exists(REF_GEN), reason="reference objects not built (no /root/reference)")
def test_llmq_writer_round_trips_through_reference_loader(tmp_path):
    """The tests' LLMQ writer is read back by the reference's own q_llama_model_load
    (llama.c:603-657) into the same weights."""
    m = O.Model(TINY, 10000.0, seed=1234)
    try:
        path = tmp_path / "tiny.llmq"
        O.write_llmq(m, str(path))
        out = subprocess.run([REF_GEN, str(tmp_path), "llmqhash", str(path)], capture_output=True, text=True,
                             check=True)
        assert int(out.stdout.strip(), 16) == m.hash()
    finally:
        m.close()


def _edge_row(name):
    if name == "V1":
        return np.array([0.25], np.float32)
    if name == "flat":
        return np.full(4096, 1.5, np.float32)
    if name == "wide":
        return O.sample_row(131072, 61, 3.0, 1)
    r = O.sample_row(5000, 60, 1.0, 0)
    if name == "ninf":
        r[::3] = -np.inf
    return r


@pytest.mark.parametrize("ci", range(len(S["edge_cases"])))
def test_sample_token_edge_cases_match_reference(ci):
    c = S["edge_cases"][ci]
    row = _edge_row(c["row"])
    st = O.rng_create(2024)
    toks = []
    for _ in range(5):
        t, st = O.sample_token(row, c["t"], c["k"], c["p"], st)
        toks.append(t)
    assert toks == c["tokens"] and st == int(c["state"], 16), c
