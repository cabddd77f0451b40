"""GPU parity of the GPT-2 (GPTC) KV decode (model.c:457-520) through the C ABI:
every step's logits bit-identical to the reference's fixtures (written by the
compiled reference), the device tanhf of the GELU against the host libm on
every float input, and a checkpoint read by gpt_load decoded on the device."""
import ctypes as C
import os
import sys

import numpy as np
import pytest

import oracle_lib as O
import qlib
from conftest import golden, golden_json

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def Q():
    q = qlib.load()
    assert q.lib().qllama_device_count() > 0, "no GPU visible to the HIP library"
    return q


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_device_tanhf_matches_host_libm_everywhere(Q):
    chunk = 1 << 28
    buf = np.empty(chunk, np.float32)
    bad = 0
    for c in range(16):
        log(f"tanhf chunk {c}/16")
        assert Q.lib().qllama_test_tanhf(c * chunk, chunk, O.fptr(buf)) == 0
        bad += int(O.lib().or_tanhf_mismatches(c * chunk, chunk, O.fptr(buf)))
    assert bad == 0


def _host_model(Q, om):
    return Q.host_gpt(om.cfg, om.tensors())


@pytest.mark.parametrize("name", ["tiny", "gpt2s", "long"])
def test_gpt_decode_matches_reference(Q, name):
    meta = golden_json(f"gpt_{name}")
    om = O.GPTModel(meta["cfg"], seed=meta["seed"])
    assert om.hash() == int(meta["model_hash"], 16)
    log(f"gpt {name}: {meta['cfg']}, {len(meta['logit_hashes'])} steps")
    dec = Q.GPTDecoder(_host_model(Q, om))
    try:
        hashes = [int(h, 16) for h in meta["logit_hashes"]]
        P = len(meta["prompt"])
        exact = 0
        for i, t in enumerate(meta["prompt"]):
            lg = dec.step(t)
            exact += O.hash_f32(lg) == hashes[i]
        head = golden(f"gpt_{name}_logits_prompt_last")
        assert np.array_equal(bits(lg[:head.size]), bits(head))
        gen = []
        for s in range(len(meta["gen"])):
            nxt = int(np.argmax(lg))
            gen.append(nxt)
            lg = dec.step(nxt)
            exact += O.hash_f32(lg) == hashes[P + s]
        assert gen == meta["gen"]
        assert np.array_equal(bits(lg[:head.size]), bits(golden(f"gpt_{name}_logits_final")))
        log(f"gpt {name}: {exact}/{len(hashes)} steps bit-identical")
        assert exact == len(hashes)
    finally:
        dec.close()
        om.close()


def test_gpt_checkpoint_to_device(Q, tmp_path):
    """gpt_load of a GPTC file, then the device decode: equal to the oracle's
    steps on the same weights; resetting len restarts the cache."""
    meta = golden_json("gpt_tiny")
    om = O.GPTModel(meta["cfg"], seed=meta["seed"])
    path = tmp_path / "tiny.gptc"
    om.write_gptc(str(path))
    m = Q.gpt_load(str(path))
    dec = Q.GPTDecoder(m)
    try:
        ids = meta["prompt"][:12]
        ref = [om.step(t).copy() for t in ids]
        got = [dec.step(t).copy() for t in ids]
        assert all(np.array_equal(bits(a), bits(b)) for a, b in zip(got, ref))
        dec.reset(0)
        assert np.array_equal(bits(dec.step(ids[0])), bits(ref[0]))
    finally:
        dec.close()
        Q.lib().gpt_free(C.byref(m))
        om.close()


def test_gpt_cache_takes_another_model(Q):
    """A cache is buffers (model.c:437-448): given another model of the same shape,
    the step uses that model's weights."""
    meta = golden_json("gpt_tiny")
    a, b = O.GPTModel(meta["cfg"], seed=1234), O.GPTModel(meta["cfg"], seed=99)
    ha, hb = _host_model(Q, a), _host_model(Q, b)
    dec = Q.GPTDecoder(ha)
    try:
        ids = meta["prompt"][:6]
        for t in ids[:3]:
            assert np.array_equal(bits(dec.step(t)), bits(a.step(t)))
        dec.m = hb                      # the next steps pass model b
        dec.reset(0)
        for t in ids:
            assert np.array_equal(bits(dec.step(t)), bits(b.step(t)))
    finally:
        dec.close()
        a.close()
        b.close()


def test_gpt_weights_changed_in_place_need_a_refresh(Q):
    """The device copy of a cache's weights is made at creation (and when the
    step is given another model): weights edited in place are not seen until
    gpt_kvcache_refresh (the contract include/qgpt.h states).  The edit here is the
    final LayerNorm gain, which leaves the cached keys and values alone, so after
    the refresh every step equals the oracle's on the edited weights again."""
    meta = golden_json("gpt_tiny")
    om = O.GPTModel(meta["cfg"], seed=meta["seed"])          # the host GPT shares its arrays
    old = O.GPTModel(meta["cfg"], seed=meta["seed"])         # the same weights, never edited
    dec = Q.GPTDecoder(_host_model(Q, om))
    try:
        ids = meta["prompt"][:8]
        for t in ids[:4]:
            g = dec.step(t).copy()
            assert np.array_equal(bits(g), bits(om.step(t))) and np.array_equal(bits(g), bits(old.step(t)))
        gain = dict(om.tensors())["ln_f_gamma"]
        gain *= np.float32(1.5)                               # in place: the host GPT sees the same memory
        assert np.array_equal(dict(Q.gpt_tensors(dec.m))["ln_f_gamma"], gain)
        g = dec.step(ids[4]).copy()
        a, b = om.step(ids[4]).copy(), old.step(ids[4]).copy()
        assert np.array_equal(bits(g), bits(b)) and not np.array_equal(bits(g), bits(a))   # stale copy
        assert Q.lib().gpt_kvcache_refresh(C.byref(dec.kv), C.byref(dec.m)) == 0
        for t in ids[5:]:
            g = dec.step(t).copy()
            assert np.array_equal(bits(g), bits(om.step(t)))
            old.step(t)
    finally:
        dec.close()
        om.close()
        old.close()
