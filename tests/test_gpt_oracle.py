"""The oracle's GPT-2 (GPTC) KV decode (model.c:437-520 with layernorm.c,
activation.c's tanh GELU and matrix.c's f32 matmul), pinned against fixtures the
compiled reference wrote (gen_golden gpt), against closed forms, and the GPTC
file format against the reference's own loader and the library's host loader.
CPU only."""
import os
import struct
import subprocess

import numpy as np
import pytest

import oracle_lib as O
import qlib
from conftest import ROOT, golden, golden_json

REF_GEN = os.path.join(ROOT, "oracle", "_ref", "gen_golden")


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["tiny", "gpt2s", "long"])
def test_gpt_oracle_matches_reference(name):
    meta = golden_json(f"gpt_{name}")
    m = O.GPTModel(meta["cfg"], seed=meta["seed"])
    try:
        assert m.hash() == int(meta["model_hash"], 16)
        hashes = [int(h, 16) for h in meta["logit_hashes"]]
        P = len(meta["prompt"])
        for i, t in enumerate(meta["prompt"]):
            lg = m.step(t)
            assert O.hash_f32(lg) == hashes[i], i
        head = golden(f"gpt_{name}_logits_prompt_last")
        assert np.array_equal(bits(lg[:head.size]), bits(head))
        for s, t in enumerate(meta["gen"]):
            assert int(np.argmax(lg)) == t, s
            lg = m.step(t)
            assert O.hash_f32(lg) == hashes[P + s], P + s
        assert np.array_equal(bits(lg[:head.size]), bits(golden(f"gpt_{name}_logits_final")))
    finally:
        m.close()


def test_layernorm_closed_forms():
    g = np.linspace(0.5, 1.5, 64).astype(np.float32)
    b = np.linspace(-0.1, 0.1, 64).astype(np.float32)
    # a constant row has mean c and variance 0: every output is (0 * r) * g + b = b
    assert np.array_equal(bits(O.layernorm(np.full((1, 64), 3.25, np.float32), g, b)[0]), bits(b))
    # +a, -a alternating: the sequential mean is exactly 0 and the variance a^2
    a = np.float32(0.75)
    x = np.tile(np.array([a, -a], np.float32), 32)[None, :]
    r = np.float32(1.0) / np.sqrt(np.float32(a * a) + np.float32(1e-5), dtype=np.float32)
    want = ((x[0] - np.float32(0.0)) * r) * g + b
    assert np.array_equal(bits(O.layernorm(x, g, b)[0]), bits(want.astype(np.float32)))
    # the output does not depend on a shift of the row by a power of two (mean moves exactly)
    rng = np.random.default_rng(5)
    y = rng.integers(-64, 64, 64).astype(np.float32)
    assert np.array_equal(bits(O.layernorm(y[None], g, b)), bits(O.layernorm((y + 1024)[None], g, b)))


def test_gelu_tanh_form():
    x = np.linspace(-9, 9, 4001).astype(np.float32)
    xd = x.astype(np.float64)
    ref = 0.5 * xd * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (xd + 0.044715 * xd ** 3)))
    got = O.gelu(x)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-7)
    assert np.array_equal(O.gelu(np.float32([0.0, 30.0])), np.float32([0.0, 30.0]))   # tanh saturates at 1


@pytest.mark.skipif(not os.path.exists(REF_GEN), reason="reference objects not built (no /root/reference)")
def test_gptc_writer_round_trips_through_reference_loader(tmp_path):
    meta = golden_json("gpt_tiny")
    m = O.GPTModel(meta["cfg"], seed=meta["seed"])
    try:
        path = tmp_path / "tiny.gptc"
        m.write_gptc(str(path))
        out = subprocess.run([REF_GEN, str(tmp_path), "gpthash", str(path)], capture_output=True, text=True,
                             timeout=120)
        assert out.returncode == 0, out.stderr
        assert int(out.stdout.strip(), 16) == m.hash() == int(meta["model_hash"], 16)
    finally:
        m.close()


def test_library_gpt_load_and_save(tmp_path):
    """The library's host gpt_load reads the GPTC writer's file into the same
    tensors; gpt_save writes the same bytes back; bad files are refused with the
    reference's messages (checkpoint.c:133-170)."""
    Q = qlib.load()
    meta = golden_json("gpt_tiny")
    om = O.GPTModel(meta["cfg"], seed=meta["seed"])
    path = tmp_path / "tiny.gptc"
    om.write_gptc(str(path))
    m = Q.gpt_load(str(path))
    try:
        assert [m.vocab_size, m.d_model, m.n_heads, m.n_layers, m.d_ff, m.max_seq_len] == meta["cfg"]
        for (n1, a), (n2, b) in zip(Q.gpt_tensors(m), om.tensors()):
            assert n1 == n2 and a.shape == b.shape and np.array_equal(bits(a), bits(b)), n1
        out = tmp_path / "copy.gptc"
        assert Q.lib().gpt_save(os.fsencode(str(out)), C_ref(m)) == 0
        assert out.read_bytes() == path.read_bytes()
    finally:
        Q.lib().gpt_free(C_ref(m))
        om.close()
    data = path.read_bytes()
    bad = tmp_path / "bad.gptc"
    for blob, msg in ((data[:-4], "truncated (bad weights)"), (data[:20], "truncated (bad header)"),
                      (struct.pack("<2I", 0x43545047, 1) + data[8:], "not a v2 GPTC"),
                      (data[:8] + struct.pack("<6i", 512, 64, 5, 2, 256, 128) + data[32:], "invalid/unsupported")):
        bad.write_bytes(blob)
        code = f"import sys; sys.path.insert(0, {os.path.join(ROOT, 'tests')!r}); import qlib; " \
               f"q = qlib.load(); sys.exit(q.lib().gpt_load({str(bad).encode()!r}, q.ctypes_byref(q.GPT())))"
        r = subprocess.run(["python3", "-c", code], capture_output=True, text=True, timeout=120)
        assert r.returncode != 0 and msg in r.stderr, (msg, r.stderr)


def test_library_gpt_save_replaces_only_when_complete(tmp_path):
    """checkpoint.c:62-103: gpt_save writes path.tmp and renames it over path,
    so a save that fails leaves an existing checkpoint byte for byte as it was,
    and a good save replaces it and leaves no temporary file."""
    Q = qlib.load()
    meta = golden_json("gpt_tiny")
    om = O.GPTModel(meta["cfg"], seed=meta["seed"])
    src = tmp_path / "tiny.gptc"
    om.write_gptc(str(src))
    m = Q.gpt_load(str(src))
    try:
        target = tmp_path / "ckpt.gptc"
        old = b"an existing checkpoint" * 100
        target.write_bytes(old)
        (tmp_path / "ckpt.gptc.tmp").mkdir()           # the temporary file cannot be created
        r = subprocess.run(
            ["python3", "-c",
             f"import sys, ctypes; sys.path.insert(0, {os.path.join(ROOT, 'tests')!r}); import qlib; "
             f"q = qlib.load(); m = q.gpt_load({str(src)!r}); "
             f"sys.exit(q.lib().gpt_save({str(target).encode()!r}, ctypes.byref(m)))"],
            capture_output=True, text=True, timeout=120)
        assert r.returncode != 0 and "cannot open" in r.stderr, r.stderr
        assert target.read_bytes() == old
        (tmp_path / "ckpt.gptc.tmp").rmdir()
        assert Q.lib().gpt_save(os.fsencode(str(target)), C_ref(m)) == 0
        assert target.read_bytes() == src.read_bytes()
        assert not (tmp_path / "ckpt.gptc.tmp").exists()
    finally:
        Q.lib().gpt_free(C_ref(m))
        om.close()


def C_ref(m):
    import ctypes
    return ctypes.byref(m)
