"""GPU parity: the HIP path through the C ABI against the reference's fixtures
and the CPU oracle.  Bar: integer data and token streams bit-exact; logits within
the north-star tolerance (max-abs 1e-3, relative 1e-4) -- and reported when they
are bit-exact, which is what this implementation aims for."""
import sys

import os

import numpy as np
import pytest

import oracle_lib as O
import qlib
from conftest import golden, golden_json, have_golden

pytestmark = pytest.mark.gpu
ATOL, RTOL = 1e-3, 1e-4


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def Q():
    q = qlib.load()
    assert q.lib().qllama_device_count() > 0, "no GPU visible to the HIP library"
    return q


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


# ---- device expf vs host libm on float bit patterns -------------------------
def test_device_expf_matches_host_libm_everywhere(Q):
    chunk = 1 << 28
    buf = np.empty(chunk, np.float32)
    total_bad = 0
    for c in range(16):
        start = c * chunk
        log(f"expf chunk {c}/16 start={start:#x}")
        assert Q.lib().qllama_test_expf(start, chunk, O.fptr(buf)) == 0
        total_bad += int(O.lib().or_expf_mismatches(start, chunk, O.fptr(buf)))
    assert total_bad == 0


# ---- weights ----------------------------------------------------------------
def test_tiny_weights_match_generator(Q):
    meta = golden_json("e2e_tiny")
    m = Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        assert m.hash() == int(meta["model_hash"], 16)
    finally:
        m.close()


# ---- end to end: tiny config ------------------------------------------------
def _run_steps(m, meta, check_every=1):
    hashes = [int(h, 16) for h in meta["logit_hashes"]]
    P = len(meta["prompt"])
    exact = 0
    m.reset()
    for i, t in enumerate(meta["prompt"]):
        lg = m.step(t)
        if i % check_every == 0 or i == P - 1:
            exact += O.hash_f32(lg) == hashes[i]
    gen = []
    for s in range(meta["gen_len"]):
        nxt = int(np.argmax(m.logits[0]))
        gen.append(nxt)
        lg = m.step(nxt)
        if s % check_every == 0 or s == meta["gen_len"] - 1:
            exact += O.hash_f32(lg) == hashes[P + s]
    return gen, exact


def test_e2e_tiny_decode_matches_reference(Q):
    meta = golden_json("e2e_tiny")
    m = Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        gen, exact = _run_steps(m, meta)
        final = m.logits[0].copy()
    finally:
        m.close()
    ref_final = golden("e2e_tiny_logits_final")
    np.testing.assert_allclose(final, ref_final, atol=ATOL, rtol=RTOL)
    assert gen == meta["gen"], "greedy token stream differs from the reference"
    log(f"tiny: {exact}/{len(meta['logit_hashes'])} steps with bit-identical logits")
    assert exact == len(meta["logit_hashes"])


def test_e2e_tiny_prefill_and_device_greedy(Q):
    meta = golden_json("e2e_tiny")
    m = Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        lg = m.prefill(meta["prompt"]).copy()
        np.testing.assert_allclose(lg, golden("e2e_tiny_logits_prompt_last"), atol=ATOL, rtol=RTOL)
        assert bits_equal(lg, golden("e2e_tiny_logits_prompt_last"))
        first = int(np.argmax(lg))
        assert first == meta["gen"][0]
        out = m.generate_greedy(first, meta["gen_len"] - 1)
        assert [first] + out == meta["gen"]
        assert m.pos == len(meta["prompt"]) + meta["gen_len"] - 1
        # the cache restarts when the caller resets len (main.c:661)
        m.reset(0)
        lg2 = m.prefill(meta["prompt"]).copy()
        assert bits_equal(lg2, lg)
    finally:
        m.close()


def test_prefill_in_pieces_equals_whole_prompt(Q):
    """Prompt ingestion in pieces (batched pieces of 16 rows and more, shorter
    ones replayed step by step) continues the cache exactly: the last logits
    equal the reference's after the whole prompt, bit for bit."""
    meta = golden_json("e2e_tiny")
    m = Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        p = meta["prompt"]
        for cut in ((100,), (7, 40), (16, 17, 50, 111)):
            m.reset(0)
            prev = 0
            for c in cut + (len(p),):
                lg = m.prefill(p[prev:c]).copy()
                prev = c
            assert bits_equal(lg, golden("e2e_tiny_logits_prompt_last")), cut
    finally:
        m.close()


def _synth_layer_path(Q, meta, fused):
    """The fixture's model, with the attention half of each decode layer as one
    launch (fused) or as separate kernels (QLLAMA_NO_ATTN_LAYER at creation)."""
    if fused:
        return Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    os.environ["QLLAMA_NO_ATTN_LAYER"] = "1"
    try:
        return Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    finally:
        del os.environ["QLLAMA_NO_ATTN_LAYER"]


def _big_prefill(Q, name, fused=True):
    """The whole prompt through the batched (MFMA) prefill, then device greedy
    decoding: last prompt logits, the token stream and the final logits equal
    the reference's."""
    if not have_golden(f"e2e_{name}.json") or not have_golden(f"e2e_{name}_logits_prompt_last.npy"):
        pytest.skip(f"{name} fixture not generated")
    meta = golden_json(f"e2e_{name}")
    m = _synth_layer_path(Q, meta, fused)
    try:
        log(f"{name}: attention half of each decode layer in one launch: {m.attn_layer_active()}")
        if name in ("8b", "1b"):      # shapes the one-launch path serves (head_dim 128 and 64)
            assert m.attn_layer_active() == fused
        log(f"{name}: batched prefill of {len(meta['prompt'])} tokens")
        lg = m.prefill(meta["prompt"]).copy()
        ref = golden(f"e2e_{name}_logits_prompt_last")
        np.testing.assert_allclose(lg[:ref.size], ref, atol=ATOL, rtol=RTOL)
        assert bits_equal(lg[:ref.size], ref)
        first = int(np.argmax(lg))
        assert first == meta["gen"][0]
        # feed every generated token, as the reference run did: the device
        # loop up to gen[-2], then a decode step (which returns logits) for gen[-1]
        out = m.generate_greedy(first, meta["gen_len"] - 1)
        assert [first] + out == meta["gen"]
        final = m.step(out[-1]).copy()
    finally:
        m.close()
    head = golden(f"e2e_{name}_logits_final")
    assert bits_equal(final[:head.size], head)


@pytest.mark.parametrize("path", ["one_launch", "separate"])
def test_e2e_1b_batched_prefill_matches_reference(Q, path):
    _big_prefill(Q, "1b", fused=path == "one_launch")


@pytest.mark.parametrize("path", ["one_launch", "separate"])
def test_e2e_8b_batched_prefill_matches_reference(Q, path):
    _big_prefill(Q, "8b", fused=path == "one_launch")


# Batched prefill over head groupings G = H/KVH, head sizes and cache lengths
# the model fixtures do not reach, against the oracle's decode steps:
# (vocab, dim, layers, H, KVH, hd, hidden, max_seq, prompt length).
PF_SHAPES = [
    (512, 512, 2, 8, 8, 64, 1024, 333, 330),     # G=1; cache rows not a multiple of 8
    (512, 1024, 2, 8, 4, 128, 2048, 600, 520),   # G=2
    (512, 384, 2, 6, 2, 48, 768, 320, 317),      # G=3
    (512, 768, 2, 8, 2, 128, 1536, 300, 290),    # G=4 with dim != H*hd
    (512, 1024, 2, 16, 2, 64, 1536, 400, 397),   # G=8
    (512, 1024, 1, 8, 1, 128, 1024, 300, 297),   # G=8 at hd 128: 1024 lanes per block
    (512, 512, 1, 16, 2, 64, 512, 16384, 1100),  # two attention passes (1 GiB of scores each)
]


@pytest.mark.parametrize("path", ["outer", "valu"])
@pytest.mark.parametrize("shape", PF_SHAPES, ids=lambda s: f"H{s[3]}kv{s[4]}hd{s[5]}T{s[7]}")
def test_batched_prefill_groupings_match_oracle(Q, shape, path):
    """The prompt in two batched pieces (the second starting at an unaligned
    position), then decode steps from the cache they left: every logit vector
    equals the oracle's after the same tokens, bit for bit.  path: prompt
    attention with its products from fp32 MFMA outer products (the default) or
    from v_mul_f32 (the VALU-only kernels)."""
    cfg, n = list(shape[:8]), shape[8]
    ids = O.prompt(n, 77, cfg[0])
    cut = 37
    log(f"prefill {cfg}: {n} prompt tokens in pieces of {cut} and {n - cut}, {path} attention")
    ref = O.Model(cfg, 10000.0, seed=4321)
    m = Q.Model.synth(cfg, 10000.0, seed=4321)
    Q.lib().qllama_test_pf_valu(1 if path == "valu" else 0)
    try:
        assert m.hash() == ref.hash()
        ref_cut = None
        for i, t in enumerate(ids):
            lg = ref.step(t)
            if i == cut - 1:
                ref_cut = lg.copy()
        assert bits_equal(m.prefill(ids[:cut]), ref_cut)
        lg = m.prefill(ids[cut:]).copy()
        assert bits_equal(lg, ref.logits)
        t = int(np.argmax(lg))
        for _ in range(min(3, cfg[7] - n)):
            a = m.step(t).copy()
            assert bits_equal(a, ref.step(t))
            t = int(np.argmax(a))
    finally:
        Q.lib().qllama_test_pf_valu(0)
        m.close()
        ref.close()


def test_decode_rejects_position_past_max_seq(Q):
    # the reference leaves this to its callers (main.c:663); the library checks
    # it on the host before any device work: run in a child so the abort is seen
    import subprocess, textwrap
    code = textwrap.dedent(f"""
        import sys; sys.path.insert(0, {qlib.ROOT + '/tests'!r})
        import qlib
        q = qlib.load()
        m = q.Model.synth([64, 16, 1, 2, 1, 8, 32, 4], 10000.0)
        for t in range(5): m.step(1)
    """)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "exceeds max_seq" in r.stderr


def test_refused_device_allocation_is_an_error_not_a_crash(Q, capfd):
    """A model larger than the GPU's memory (about 440 GB of int8 weights): the
    device allocation is refused, q_llama_model_synth prints an error and
    returns nonzero (as the reference's loaders do on failure), and the library
    stays usable: a small model built afterwards decodes bit-exactly."""
    big = [128256, 16384, 200, 128, 16, 128, 32768, 64]
    with pytest.raises(RuntimeError):
        Q.Model.synth(big, 10000.0)
    assert "device allocation" in capfd.readouterr().err
    meta = golden_json("e2e_tiny")
    m = Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"])
    try:
        for i, t in enumerate(meta["prompt"][:4]):
            lg = m.step(t)
            assert O.hash_f32(lg) == int(meta["logit_hashes"][i], 16), i
    finally:
        m.close()


# ---- quant.h API ------------------------------------------------------------
@pytest.mark.parametrize("case", ["a", "b"])
def test_quantize_int8_percol_matches_reference(Q, case):
    q, s = Q.quantize_int8_percol(golden(f"quant_{case}_w"))
    assert np.array_equal(q, golden(f"quant_{case}_q"))
    assert bits_equal(s, golden(f"quant_{case}_scale"))


def test_dequantize_matches_reference(Q):
    assert bits_equal(Q.dequantize_int8_percol(golden("quant_b_q"), golden("quant_b_scale")), golden("quant_b_deq"))


@pytest.mark.parametrize("name", ["qmm_1x64x48", "qmm_3x300x17", "qmm_8x256x96"])
def test_qmatmul_small_matches_reference(Q, name):
    meta = golden_json("ops")[name]
    K, N = meta["K"], meta["N"]
    A = golden(f"{name}_A")
    w = O.synth(K * N, meta["seed"], 5010, 0.02).reshape(K, N)    # the fixture's fp32 weight
    q, s = Q.quantize_int8_percol(w)
    assert np.array_equal(q, golden(f"{name}_Wq")) and bits_equal(s, golden(f"{name}_Ws"))
    W = Q.QWeight(w)
    try:
        Cg = Q.qmatmul(A, W)
    finally:
        W.close()
    ref = golden(f"{name}_C")
    np.testing.assert_allclose(Cg, ref, atol=ATOL, rtol=RTOL)
    assert bits_equal(Cg, ref)


@pytest.mark.parametrize("M,K,N", [(16, 64, 48), (130, 300, 200), (300, 1000, 517), (1024, 4096, 384)])
def test_qmatmul_many_rows_matches_oracle(Q, M, K, N):
    """16 rows and more go through the MFMA GEMM: bit-identical to the C
    restatement of quant.c:60-85 (int32 accumulation is exact), including
    partial row/column tiles and K that is not a multiple of the 64-byte step."""
    rng = np.random.default_rng(M * 7 + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[3] = 0.0                                   # an all-zero row: scale 1
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    q, s = O.quantize(w)
    W = Q.QWeight(w)
    try:
        Cg = Q.qmatmul(A, W)
    finally:
        W.close()
    ref = O.qmatmul(A, q, s)
    assert bits_equal(Cg, ref)


@pytest.mark.parametrize("M,K,N", [(2, 64, 48), (5, 300, 200), (16, 1000, 517), (11, 14336, 96),
                                   (8, 4096, 4096), (2, 2048, 33), (3, 4096, 1001), (4, 8192, 96), (6, 14336, 257),
                                   (8, 512, 70001), (3, 256, 140000), (16, 128, 65536),
                                   (7, 1024, 5000), (2, 8192, 77), (5, 3072, 70001), (8, 14336, 4096),
                                   (8, 8192, 1000), (6, 2048, 333)])
def test_qmatmul_few_rows_matches_oracle(Q, M, K, N):
    """2..16 rows.  2..8 rows with K a multiple of 1024 up to 8192 go through
    the whole-row kernel (k_gemv_rows: 1..8 waves a block, 2, 4 or 8 rows a
    pass, N not a multiple of its 8-channel groups); other vocabulary-sized
    outputs (N >= 65536) through the persistent skinny kernel (k_gemv_skinny: K
    split over 2 waves or not, N odd), the rest through the per-block skinny
    kernel (k_gemv_mfma, including K that is not a multiple of the 64-byte
    step): all bit-identical to quant.c:60-85."""
    rng = np.random.default_rng(M * 131 + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[M - 1] = 0.0                               # an all-zero row: scale 1
    w = (rng.standard_normal((K, N)) * 0.02).astype(np.float32)
    q, s = O.quantize(w)
    W = Q.QWeight(w)
    try:
        Cg = Q.qmatmul(A, W)
    finally:
        W.close()
    assert bits_equal(Cg, O.qmatmul(A, q, s))


def test_qacc_columns_exact(Q):
    rng = np.random.default_rng(3)
    qa = rng.integers(-127, 128, 300).astype(np.int8)
    qw = rng.integers(-127, 128, (300, 77)).astype(np.int8)
    acc = Q.qacc_columns(qa, qw)
    assert np.array_equal(acc.astype(np.int64), qa.astype(np.int64) @ qw.astype(np.int64))


@pytest.mark.parametrize("si", [0, 1, 2, 3])
def test_gemv_op_level_matches_reference(Q, si):
    meta = golden_json("ops")[f"gemv_{si}"]
    M, K = meta["M"], meta["K"]
    log(f"gemv shape {si}: M={M} K={K}")
    wf = O.synth(K * M, 1234, 1000 + si, 0.02).reshape(K, M)
    W = Q.QWeight(wf)
    del wf
    try:
        for b in (1, 8):
            x = O.synth(b * K, 1234, 2000 + si, 1.0).reshape(b, K)
            y = Q.qmatmul(x, W)
            assert O.hash_f32(y) == int(meta[f"b{b}_hash"], 16), f"batch {b}"
            np.testing.assert_allclose(y.ravel()[:256], golden(f"gemv_{si}_b{b}_head"), atol=ATOL, rtol=RTOL)
    finally:
        W.close()


# ---- the decode GEMV's own rmsnorm prologue (rmsnorm.c:7-21 inside k_gemv_dec) --
@pytest.mark.parametrize("dm", [2048, 4096])
def test_fused_rmsnorm_gemv_matches_reference(Q, dm):
    """Every block of the QKV and gate|up decode GEMVs normalizes and quantizes
    the residual row itself.  On the committed rmsnorm fixtures (rows with
    non-unit gains) the plain GEMV equals rmsnorm.c's output fed to quant.c's
    qmatmul bit for bit, and the SwiGLU GEMV equals the oracle's gate and up
    outputs combined by llama.c:583-587's expression."""
    xs, g, ys = golden(f"rms_{dm}_x"), golden(f"rms_{dm}_g"), golden(f"rms_{dm}_y")
    N = 1536
    w = O.synth(dm * N, 1234, 6000 + dm, 0.02).reshape(dm, N)
    q, s = O.quantize(w)
    W = Q.QWeight(w)
    try:
        for r in range(xs.shape[0]):
            out = Q.norm_gemv(xs[r], g, W, mode=0)
            assert bits_equal(out, O.qmatmul(ys[r:r + 1], q, s)[0]), f"row {r}"
            h = Q.norm_gemv(xs[r], g, W, mode=2)
            gu = O.qmatmul(ys[r:r + 1], q, s)[0]
            gate, up = gu[:N // 2], gu[N // 2:]
            ref = (gate * (np.float32(1.0) / (np.float32(1.0) + np.exp(-gate)))) * up
            np.testing.assert_allclose(h, ref, atol=ATOL, rtol=RTOL)
    finally:
        W.close()


# ---- op-level decode attention ---------------------------
@pytest.mark.parametrize("T", [1, 512, 2048, 8192])
def test_gqa_decode_matches_reference(Q, T):
    H, KVH, hd = 32, 8, 128
    if T == 8192:
        if not have_golden("gqa_T8192_o.npy"):
            pytest.skip("context-8192 fixture not generated")
        meta = golden_json("gqa8192")[f"gqa_T{T}"]
    else:
        meta = golden_json("ops")[f"gqa_T{T}"]
    case = meta["case"]
    Qm = O.synth(T * H * hd, 31, 3000 + case, 1.0).reshape(T, H * hd)
    q = O.rope(Qm[T - 1:T], H, 500000.0, T - 1)[0]
    del Qm
    K = O.rope(O.synth(T * KVH * hd, 31, 3100 + case, 1.0).reshape(T, KVH * hd), KVH, 500000.0, 0)
    V = O.synth(T * KVH * hd, 31, 3200 + case, 1.0).reshape(T, KVH * hd)
    assert O.hash_f32(K) == int(meta["k_hash"], 16)
    o = np.zeros(H * hd, np.float32)
    assert Q.lib().qllama_gqa_decode(O.fptr(q), O.fptr(K), O.fptr(V), T, H, KVH, hd, O.fptr(o)) == 0
    ref = golden(f"gqa_T{T}_o")
    np.testing.assert_allclose(o, ref, atol=ATOL, rtol=RTOL)
    assert bits_equal(o, ref)


@pytest.mark.parametrize("T", [300, 700, 1300, 1800, 2300, 2800, 3500, 6000])
def test_gqa_decode_softmax_bands_match_oracle(Q, T):
    """The decode attention at a context in each band of softmax terms a thread
    (1, 2, 3, 4, 5, 6, 8, 16 of 512 threads): bit-identical to the C restatement
    of llama.c:554-576."""
    H, KVH, hd = 32, 8, 128
    rng = np.random.default_rng(900 + T)
    q = rng.standard_normal(H * hd, dtype=np.float32)
    K = rng.standard_normal((T, KVH * hd), dtype=np.float32)
    V = rng.standard_normal((T, KVH * hd), dtype=np.float32)
    o = np.zeros(H * hd, np.float32)
    assert Q.lib().qllama_gqa_decode(O.fptr(q), O.fptr(K), O.fptr(V), T, H, KVH, hd, O.fptr(o)) == 0
    assert bits_equal(o, O.attn_decode(q, K, V, T - 1, H, KVH, hd))


def test_long_context_decode_matches_oracle(Q):
    """A 2990-token prompt through the batched prefill, then decode steps at
    2990-3089 cached positions through the one-launch attention (its 6- and
    8-terms-a-thread softmax bands): every logit vector equals the oracle's
    decode step after the same tokens, bit for bit."""
    cfg = [512, 2048, 1, 32, 8, 64, 512, 4096]
    n, extra = 2990, 100
    ids = O.prompt(n, 78, cfg[0])
    ref = O.Model(cfg, 500000.0, seed=4321)
    m = Q.Model.synth(cfg, 500000.0, seed=4321)
    try:
        assert m.hash() == ref.hash()
        assert m.attn_layer_active()
        log(f"oracle: {n} decode steps")
        for t in ids:
            ref.step(t)
        lg = m.prefill(ids).copy()
        assert bits_equal(lg, ref.logits)
        t = int(np.argmax(lg))
        for s in range(extra):
            a = m.step(t).copy()
            assert bits_equal(a, ref.step(t)), f"decode step at position {n + s}"
            t = int(np.argmax(a))
    finally:
        m.close()
        ref.close()


# ---- 1B and 8B shaped models --------------------------------------------------
def _big_e2e(Q, name):
    if not have_golden(f"e2e_{name}.json"):
        pytest.skip(f"{name} fixture not generated")
    meta = golden_json(f"e2e_{name}")
    log(f"{name}: building the model on the device")
    m = Q.Model.synth(meta["cfg"], meta["rope_base"], seed=meta["seed"], tied=bool(meta["tied"]))
    try:
        assert m.hash() == int(meta["model_hash"], 16)
        log(f"{name}: attention half of each decode layer in one launch: {m.attn_layer_active()}")
        assert m.attn_layer_active()          # the 1B and 8B shapes take the one-launch path
        log(f"{name}: weights match; decoding {len(meta['argmax'])} steps")
        gen, exact = _run_steps(m, meta)
        final = m.logits[0].copy()
    finally:
        m.close()
    head = golden(f"e2e_{name}_logits_final")
    np.testing.assert_allclose(final[:head.size], head, atol=ATOL, rtol=RTOL)
    assert gen == meta["gen"]
    log(f"{name}: {exact}/{len(meta['logit_hashes'])} steps with bit-identical logits")
    assert exact == len(meta["logit_hashes"])


def test_e2e_1b_matches_reference(Q):
    _big_e2e(Q, "1b")


def test_e2e_8b_matches_reference(Q):
    _big_e2e(Q, "8b")


@pytest.mark.gpu
@pytest.mark.parametrize("mode,M,N,kpad,bias", [
    (0, 40, 200, 1024, True),      # plain + bias (QKV-like), 2 tiles
    (1, 100, 96, 2048, False),     # residual add
    (2, 64, 150, 1024, False),     # SwiGLU over 2N weight rows
    (1, 300, 64, 8192, False),     # long K: 256-row tiles, 16 splits
    (2, 17, 700, 4096, False),
    (0, 24, 6144, 4096, True),     # the 8B QKV at a short prompt: a last split shorter than the others
    (1, 20, 1024, 14336, False),   # K = 14336 (the down projection's), 224 K steps
])
def test_split_k_gemm_same_bits(Q, mode, M, N, kpad, bias):
    """The prompt GEMM with K split over extra blocks (int32 partial sums, then
    the epilogue) gives the unsplit GEMM's bits; for the plain and residual
    epilogues both equal the float32 restatement of quant.c:60-85's scaling
    over the exact integer sums."""
    import ctypes as C
    rng = np.random.default_rng(7000 + 31 * mode + M)
    wrows = 2 * N if mode == 2 else N
    A = rng.integers(-127, 128, (M, kpad), dtype=np.int8)
    W = rng.integers(-127, 128, (wrows, kpad), dtype=np.int8)
    a_s = rng.uniform(1e-4, 1e-2, M).astype(np.float32)
    w_s = rng.uniform(1e-4, 1e-2, wrows).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32) if bias else None
    init = rng.standard_normal((M, N)).astype(np.float32)
    o1, o2, splits = init.copy(), init.copy(), C.c_int(0)
    f = Q.lib().qllama_test_gemm_split
    f.restype = C.c_int
    f.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p,
                  C.c_void_p, C.c_void_p, C.POINTER(C.c_int)]
    p = lambda x: None if x is None else x.ctypes.data_as(C.c_void_p)
    assert f(mode, p(A), p(a_s), p(W), p(w_s), M, N, kpad, p(b), p(o1), p(o2), C.byref(splits)) == 0
    assert splits.value >= 2, "the shape was meant to split K"
    nkt = (kpad + 63) // 64
    log(f"split K: {splits.value} splits of {nkt} K steps (last split shorter: {nkt % splits.value != 0})")
    if (mode, M, N, kpad) == (0, 24, 6144, 4096):
        assert nkt % splits.value != 0, "this case was meant to have a shorter last split"
    assert o1.tobytes() == o2.tobytes()
    if mode != 2:
        acc = A.astype(np.int64) @ W.astype(np.int64).T
        c = (a_s[:, None] * w_s[None, :]) * acc.astype(np.float32)
        want = init + c if mode == 1 else (c + b if bias else c)
        assert np.array_equal(o1.view(np.uint32), want.astype(np.float32).view(np.uint32))
