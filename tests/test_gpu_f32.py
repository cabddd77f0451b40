"""GPU fp32 (LLMA) decode path through the C ABI (llama_kv_create /
llama_decode_step) against the fixtures the compiled reference wrote
(gen_golden e2e_f32) and against the oracle's k-order matmul.  Bar: token
streams and logits bit-exact (north-star tolerance reported too)."""
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


def gpu_model(Q, ref, cfg, base):
    return Q.FModel(Q.host_model(cfg, base, 1e-5, ref.tensors()))


@pytest.mark.parametrize("name", ["tiny", "mid"])
def test_f32_decode_matches_reference(Q, name):
    meta = golden_json(f"e2e_f32_{name}")
    ref = O.FModel(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    try:
        assert ref.hash() == int(meta["model_hash"], 16)
        g = gpu_model(Q, ref, meta["cfg"], meta["rope_base"])
        try:
            hashes = [int(h, 16) for h in meta["logit_hashes"]]
            P = len(meta["prompt"])
            for i, t in enumerate(meta["prompt"]):
                log(f"{name} prompt step {i}")
                lg = g.step(t)
                assert O.hash_f32(lg) == hashes[i], i
            np.testing.assert_allclose(lg, golden(f"e2e_f32_{name}_logits_prompt_last"), atol=1e-3, rtol=1e-4)
            assert np.array_equal(bits(lg), bits(golden(f"e2e_f32_{name}_logits_prompt_last")))
            for s, t in enumerate(meta["gen"]):
                assert int(np.argmax(lg)) == t, s
                lg = g.step(t)
                assert O.hash_f32(lg) == hashes[P + s], P + s
            assert np.array_equal(bits(lg), bits(golden(f"e2e_f32_{name}_logits_final")))
        finally:
            g.close()
    finally:
        ref.close()


@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096), (4096, 1024), (300, 17), (1000, 130), (129, 16)])
def test_f32_gemv_rows_match_oracle(Q, shape):
    """The fp32 GEMV at (K, N) through a one-layer model whose down projection
    has K inputs and whose head has N outputs: every step's logits bit for bit
    against the oracle (k-order chains over partial tiles, partial column
    blocks, the 14336-input down projection of the 8B shape)."""
    K, N = shape
    dm = 16 * ((K + 15) // 16) if K % 16 else K
    cfg = [N if N >= 16 else 16, min(dm, 4096), 1, 4, 2, 32, max(K, 64), 32]
    ref = O.FModel(cfg, 10000.0, seed=7)
    try:
        g = gpu_model(Q, ref, cfg, 10000.0)
        try:
            for t in [1, 5, 2, 9]:
                r = ref.step(t % cfg[0]).copy()
                o = g.step(t % cfg[0]).copy()
                assert np.array_equal(bits(o), bits(r)), shape
        finally:
            g.close()
    finally:
        ref.close()


def test_two_caches_share_one_device_copy(Q):
    meta = golden_json("e2e_f32_tiny")
    ref = O.FModel(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        host = Q.host_model(meta["cfg"], meta["rope_base"], 1e-5, ref.tensors())
        a, b = Q.FModel(host), Q.FModel(host)
        try:
            la = [a.step(t).copy() for t in meta["prompt"][:6]]
            a.close()                                    # b keeps the device copy alive
            lb = [b.step(t).copy() for t in meta["prompt"][:6]]
            for x, y in zip(la, lb):
                assert np.array_equal(bits(x), bits(y))
            b.reset(0)
            assert np.array_equal(bits(b.step(meta["prompt"][0])), bits(la[0]))
        finally:
            a.close()
            b.close()
    finally:
        ref.close()


def test_cli_f32_branch_matches_reference(Q, tmp_path):
    """qllama-cli on an LLMA file: the `llama` command's f32 branch (main.c:686-700)
    with decode and sampling on the GPU, against the compiled reference's loop."""
    import os
    import subprocess
    from conftest import ROOT
    cli = os.path.join(ROOT, "llm-project_amd", "qllama-cli")
    S = golden_json("sample")["cli_f32"]
    meta = golden_json("e2e_f32_tiny")
    ref = O.FModel(meta["cfg"], meta["rope_base"], seed=S["seed"])
    try:
        path = str(tmp_path / "tiny.llma")
        ref.write_llma(path)
    finally:
        ref.close()
    stdin = "".join(" ".join(str(t) for t in ln["prompt"]) + "\n" for ln in S["lines"])
    expect = []
    for ln in S["lines"]:
        expect += [f"t {t}" for t in ln["gen"]]
        expect.append("gen: " + " ".join(str(t) for t in ln["prompt"] + ln["gen"]))
    log("running qllama-cli on an LLMA file")
    out = subprocess.run([cli, "llama", path, str(S["n_new"])], input=stdin.encode(), capture_output=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr.decode()
    assert out.stdout.decode().splitlines() == expect


@pytest.mark.parametrize("name", ["tiny", "mid"])
def test_f32_forward_matches_reference(Q, name):
    """llama_model_forward on the GPU against the reference's batched forward rows."""
    meta = golden_json(f"e2e_f32_{name}")
    ref = O.FModel(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    try:
        g = gpu_model(Q, ref, meta["cfg"], meta["rope_base"])
        try:
            L = g.forward(meta["prompt"])
            assert [f"{O.hash_f32(r):016x}" for r in L] == meta["forward_hashes"]
            assert g.pos == 0                       # the caller's cache is untouched
        finally:
            g.close()
    finally:
        ref.close()


def perturb(ref, seed):
    """Nonzero q/k/v biases and norm gains other than 1 (llama.c:319-321, rmsnorm.c:18)."""
    rng = np.random.default_rng(seed)
    for name, t in ref.tensors():
        if name in ("b_q", "b_k", "b_v"):
            t[:] = rng.standard_normal(t.shape).astype(np.float32) * np.float32(0.1)
        if name in ("attn_norm", "ffn_norm", "final_norm"):
            t[:] = (1.0 + rng.standard_normal(t.shape) * 0.2).astype(np.float32)


def test_f32_forward_two_passes_match_oracle(Q):
    """The batched forward over 2100 rows, so each layer takes two passes (2048 +
    52 rows) and the second pass attends to the first's cache rows; biases, norm
    gains and an FFN width of 250 (not a multiple of 4: the GEMM's scalar loads).
    Every row bit for bit against the oracle's decode step at that position."""
    cfg = [700, 128, 2, 4, 2, 64, 250, 2112]
    n = 2100
    ref = O.FModel(cfg, 10000.0, seed=41)
    try:
        perturb(ref, 9)
        ids = [int(t) for t in np.random.default_rng(3).integers(0, cfg[0], n)]
        g = gpu_model(Q, ref, cfg, 10000.0)
        try:
            log("forward of 2100 rows")
            L = g.forward(ids)
        finally:
            g.close()
        for i, t in enumerate(ids):
            r = ref.step(t)
            assert np.array_equal(bits(L[i]), bits(r)), i
    finally:
        ref.close()


def test_f32_forward_past_max_seq_matches_oracle(Q):
    """seq_len above the model's max_seq (the reference's forward has no such
    bound, llama.c:167-186): positions 16 .. 39 take RoPE tables made for the
    call.  Rows against the oracle's decode steps on the same weights with room
    for 64 positions."""
    cfg16 = [500, 192, 2, 6, 2, 48, 320, 16]
    cfg64 = cfg16[:7] + [64]
    ref = O.FModel(cfg64, 10000.0, seed=17)
    try:
        ids = [int(t) for t in np.random.default_rng(4).integers(0, 500, 40)]
        g = gpu_model(Q, ref, cfg16, 10000.0)
        try:
            L = g.forward(ids)
        finally:
            g.close()
        for i, t in enumerate(ids):
            assert np.array_equal(bits(L[i]), bits(ref.step(t))), i
    finally:
        ref.close()


def test_f32_forward_batched_equals_steps(Q, monkeypatch):
    """The batched forward and the decode-step replay (QLLAMA_FORWARD_STEPS=1)
    give the same bits on the mid fixture's model."""
    meta = golden_json("e2e_f32_mid")
    ref = O.FModel(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    try:
        g = gpu_model(Q, ref, meta["cfg"], meta["rope_base"])
        try:
            ids = list(meta["prompt"]) * 3
            a = g.forward(ids)
            monkeypatch.setenv("QLLAMA_FORWARD_STEPS", "1")
            b = g.forward(ids)
            assert np.array_equal(bits(a), bits(b))
        finally:
            g.close()
    finally:
        ref.close()


def test_f32_nonzero_biases_and_gains_match_oracle(Q):
    """Biases (Qwen-style checkpoints, llama.c:319-321) and norm gains other than 1
    (rmsnorm.c:18) through the fp32 step, bit for bit against the oracle."""
    cfg = [3000, 256, 2, 8, 2, 32, 512, 64]
    ref = O.FModel(cfg, 10000.0, seed=31)
    try:
        perturb(ref, 5)
        g = gpu_model(Q, ref, cfg, 10000.0)
        try:
            for t in [3, 17, 2999, 0, 42, 7]:
                a = g.step(t).copy()
                b = ref.step(t).copy()
                assert np.array_equal(bits(a), bits(b)), t
        finally:
            g.close()
    finally:
        ref.close()
