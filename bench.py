#!/usr/bin/env python3
"""Decode / prefill benchmark of the MI355X int8 LLaMA path (one GPU).

Workload (the one the headline metric is quoted on):
Llama-3-8B-shaped model with seeded synthetic weights (fp32 N(0, 0.02) quantized
per output channel to int8), a 2048-token uniform-random prompt, then greedy
decode steps.  A "step" is one decode token through the whole model.  Everything
the timed region touches is already resident in HBM.

Prints one JSON line (rank 0) with decode tok/s, the dominant kernel's roofline
(the W8A8 GEMV, timed with HIP events on the library's stream), prefill tok/s
with the MFMA GEMMs' roofline, decode with on-device sampling, and the CPU
oracle timed on this host's cores on the same weights.

`--path f32` measures the fp32 (LLMA) decode path instead (llama_decode_step on
a host LlamaModel of numpy N(0, 0.02) weights), with the f32 GEMV's roofline.
"""
import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

CONFIGS = {
    # cfg = vocab, d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq; rope base; tied; prefill
    "8b": ([128256, 4096, 32, 32, 8, 128, 14336, 2560], 500000.0, False, 2048),
    "1b": ([128256, 2048, 16, 32, 8, 64, 8192, 768], 500000.0, True, 512),
    "tiny": ([32000, 288, 6, 6, 2, 48, 768, 256], 10000.0, False, 128),
}
METRIC = "decode tok/s + % HBM roofline, 8B-shape int8 LLaMA (1 GPU); prefill tok/s"
HBM_PEAK_GBS = 8000.0
INT8_MFMA_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
F32_MFMA_TFLOPS = 157.3           # MI355X published fp32 peak
F32_VALU_TFLOPS = 78.6            # 256 CUs x 128 lanes x 2.4 GHz: unpacked, unfused fp32 ops (the published 157.3 counts an FMA as 2)
# HBM bytes per GEMV dispatch measured by rocprofv3 FETCH_SIZE / WRITE_SIZE runs
# (scaled by a plain copy of known size), written by llm-project_amd/profsum.py
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "k_gemv_dec_traffic_8b.json")


def load_qllama():
    import importlib.util
    spec = importlib.util.spec_from_file_location("qllama", os.path.join(ROOT, "llm-project_amd", "qllama.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def gemv_bytes(cfg):
    """Algorithmic HBM bytes of each GEMV launch per token: int8 weights + fp32
    scales + the activation row (int8; fp32 for Wo, which quantizes it itself)
    + fp32 outputs (read too where residual)."""
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    n_qkv = qd + 2 * kvd

    def g(N, K, extra_per_row):
        return N * K + 4 * N + K + extra_per_row * N

    return {
        "gemv_qkv": (L, g(n_qkv, dm, 4 + 4)),      # out + bias
        "gemv_o": (L, g(dm, qd, 8) + 3 * qd),      # fp32 activation; residual read + write
        "gemv_gate_up": (L, g(2 * ff, dm, 4)),
        "gemv_down": (L, g(dm, ff, 8)),
        "gemv_head": (1, g(vocab, dm, 4)),
    }


def prefill_gemm_ops(cfg, P):
    """int8 multiply-adds x 2 of the prompt GEMMs (QKV, O, gate|up, down per layer)."""
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    return 2 * P * L * (dm * (qd + 2 * kvd) + qd * dm + 2 * dm * ff + ff * dm)


def decode_bytes(cfg, t):
    """Algorithmic HBM bytes of one decode token attending over t cached rows."""
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    w = L * (dm * (qd + 2 * kvd) + qd * dm + 2 * dm * ff + ff * dm) + dm * vocab
    scales = 4 * (L * ((qd + 2 * kvd) + dm + 2 * ff + dm) + vocab)
    f32 = 4 * (2 * L * dm + L * (qd + 2 * kvd) + dm)
    kv = 2 * L * kvd * 4 * t + 2 * L * kvd * 4
    return w + scales + f32 + kv + dm


def cpu_baseline(Q, gm, cfg, base, pos0, seconds, prefill_tokens=0, prefill_seconds=0.0):
    """The CPU oracle (a C11 restatement of the reference decode step, threaded
    like the reference, matrix.c:110-117) on this host's cores: same weights,
    exported from the device; cache rows N(0,1) up to pos0.

    decode: steps timed at positions pos0.. until `seconds` of work.
    prefill (when prefill_tokens > 0): the reference's prompt ingestion is one
    decode step per token (main.c:662), so its rate is 1 / the mean step time
    over positions 0 .. prefill_tokens-1; a bounded sample of steps at evenly
    spaced positions of that range (each from a cache holding the rows before
    it) until `prefill_seconds` of work."""
    import oracle_lib as O
    nthreads = len(os.sched_getaffinity(0))
    O.lib().or_set_threads(nthreads)
    om = O.Model(cfg, base, synth=False)
    L = cfg[2]

    def export(qt, oqt):
        if Q.lib().q_llama_tensor_export(C.byref(qt), oqt.q, oqt.scale) != 0:
            raise RuntimeError("tensor export failed")

    export(gm.m.wte, om.m.wte)
    export(gm.m.lm_head, om.m.lm_head)
    for l in range(L):
        gb, ob = gm.m.blocks[l], om.m.blocks[l]
        for n in ("Wq", "Wk", "Wv", "Wo", "Wgate", "Wup", "Wdown"):
            export(getattr(gb, n), getattr(ob, n))
    kvd = cfg[4] * cfg[5]
    per = cfg[7] * kvd
    rng = np.random.default_rng(7)
    fill = max(pos0, prefill_tokens)
    for arr_ptr in (om.kv.k, om.kv.v):
        view = np.ctypeslib.as_array(arr_ptr, shape=(L * per,))
        for l in range(L):
            view[l * per:l * per + fill * kvd] = rng.standard_normal(fill * kvd, dtype=np.float32)
    om.reset(pos0)
    om.step(1)                                   # warm-up
    times = []
    t_start = time.perf_counter()
    tok = int(np.argmax(om.logits))
    while len(times) < 2 or (time.perf_counter() - t_start < seconds and len(times) < 64):
        t0 = time.perf_counter()
        lg = om.step(tok)
        times.append(time.perf_counter() - t0)
        tok = int(np.argmax(lg))
    pf = None
    if prefill_tokens > 0:
        ptimes, positions = [], []
        t_start = time.perf_counter()
        for k in range(64):
            p = (k * 37 % 64) * prefill_tokens // 64          # evenly spaced positions, visited in a spread order
            om.reset(p)
            t0 = time.perf_counter()
            om.step(tok)
            ptimes.append(time.perf_counter() - t0)
            positions.append(p)
            if len(ptimes) >= 4 and time.perf_counter() - t_start >= prefill_seconds:
                break
        mean = statistics.mean(ptimes)
        pf = {"tok_s": round(1.0 / mean, 4), "prompt_tokens": prefill_tokens,
              "sample": f"{len(ptimes)} decode steps at positions {sorted(positions)[0]}..{sorted(positions)[-1]} "
                        f"spread over the {prefill_tokens}-token prompt (the reference ingests a prompt one decode "
                        f"step per token, main.c:662); mean step {mean * 1e3:.2f} ms"}
    om.close()
    med = statistics.median(times)
    cpu_model, libc = host_info()
    out = {"value": round(1.0 / med, 4), "unit": "tok/s", "cores": nthreads, "kind": "port",
           "cpu_model": cpu_model, "libc": libc, "lscpu": lscpu_info(),
           "sample": f"{len(times)} decode steps at positions {pos0 + 1}..{pos0 + len(times)} of the same "
                     f"model (weights copied from the GPU, earlier cache rows N(0,1)); median step "
                     f"{med * 1e3:.1f} ms, oracle/liboracle with {nthreads} threads"}
    if pf:
        out["prefill"] = pf
    return out


def lscpu_info():
    """The host CPU as lscpu names it (model, BIOS model name, family/model/stepping,
    sockets and cores), for the CPU baseline's context."""
    import subprocess
    keys = ("Vendor ID", "Model name", "BIOS Model name", "CPU family", "Model", "Stepping", "Socket(s)",
            "Core(s) per socket", "Thread(s) per core", "NUMA node(s)", "CPU max MHz", "L3 cache")
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    info = {}
    for line in out.splitlines():
        k, _, v = line.partition(":")
        if k.strip() in keys:
            info[k.strip()] = v.strip()
    return info or None


def host_info():
    """CPU model and C library of this host (the CPU baseline's context)."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        libc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        libc = None
    return model, libc


GEMV_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]   # (M out, K in)


def op_gemv(Q, reps=100):
    """BASELINE's op-level int8 GEMV: W int8 (K, M) per-channel from the
    generator's N(0, 0.02) (the parity fixtures' weights), x fp32 N(0, 1) rows,
    batch 1 and 8, inputs resident in HBM.  Per call: activation quantization +
    product; the product kernel's own duration gives the roofline.  "cold":
    every call behind a 512 MB read (weights in neither L2 nor the 256 MB
    memory-side cache, as in a model's decode step); "warm": back-to-back calls
    on the same weights (the smaller shapes then come from the memory-side
    cache).  Kernel durations are per launch on a drained stream."""
    out = []
    for si, (M, K) in enumerate(GEMV_SHAPES):
        W = Q.lib().qtensor_synth(K, M, 1234, 1000 + si, 0.02)
        try:
            for B in (1, 8):
                row = {"M": M, "K": K, "batch": B,
                       "kernel": "k_gemv_dec" if B == 1 else "k_gemv_rows" if K % 1024 == 0 and K <= 8192
                       else "k_gemv_skinny" if M >= 65536 else "k_gemv_mfma"}
                op_bytes = M * K + 4 * M + 4 * B * K + 4 * B * M          # algorithmic bytes: weights, scales, x, y
                kern_bytes = M * K + 4 * M + B * K + 4 * B * M            # the product kernel reads int8 rows
                for temp in ("cold", "warm"):
                    Q.bench_cold(temp == "cold")
                    call, prod, quant = C.c_double(0), C.c_double(0), C.c_double(0)
                    if Q.lib().qllama_bench_qmatmul(C.byref(W), B, reps, C.byref(call), C.byref(prod), C.byref(quant)):
                        raise RuntimeError("qllama_bench_qmatmul failed")
                    gbs = kern_bytes / (prod.value * 1e-6) / 1e9
                    row[temp] = {"us_per_call": round(call.value, 3), "us_product": round(prod.value, 3),
                                 "us_quant": round(quant.value, 3),
                                 "call_gbs": round(op_bytes / (call.value * 1e-6) / 1e9, 1),
                                 "product_gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
                out.append(row)
        finally:
            Q.bench_cold(False)
            Q.lib().qtensor_free(C.byref(W))
    return out


def op_gqa(Q, reps=50):
    """BASELINE's op-level decode attention: 32 query / 8 KV heads, head_dim 128,
    RoPE theta 500000 applied on the device to q and the new k row, fp32 cache of
    N(0, 1) at contexts 1, 512, 2048, 8192; exact and fast modes.  "cold": each
    call behind a 512 MB read (the cache in neither L2 nor the memory-side
    cache); "warm": back-to-back calls (caches up to 256 MB then come from the
    memory-side cache).  Kernel durations are per launch on a drained stream."""
    H, KVH, hd = 32, 8, 128
    rng = np.random.default_rng(11)
    out = []
    for T in (1, 512, 2048, 8192):
        q = rng.standard_normal(H * hd, dtype=np.float32)
        k = rng.standard_normal((T, KVH * hd), dtype=np.float32)
        v = rng.standard_normal((T, KVH * hd), dtype=np.float32)
        nbytes = 2 * T * KVH * hd * 4
        for mode, name in ((Q.MODE_EXACT, "exact"), (Q.MODE_FAST, "fast")):
            row = {"T": T, "mode": name}
            for temp in ("cold", "warm"):
                Q.bench_cold(temp == "cold")
                try:
                    _, _, us = Q.gqa_decode(q, k, v, H, KVH, hd, mode=mode, rope_base=500000.0, reps=reps)
                    # kernel time per call: every launch's own events (one warm-up call + reps)
                    Q.profile(Q.PROFILE_COLD if temp == "cold" else Q.PROFILE_SERIAL)
                    Q.gqa_decode(q, k, v, H, KVH, hd, mode=mode, rope_base=500000.0, reps=reps)
                    prof = Q.profile_read()
                    Q.profile(False)
                finally:
                    Q.bench_cold(False)
                kern = {c: v_[0] * 1e3 for c, v_ in prof.items() if c.startswith("attn")}
                kus = sum(kern.values())
                row[temp] = {"us_per_call": round(us, 3),
                             "kernel_us": {c: round(x, 3) for c, x in sorted(kern.items())},
                             "gbs": round(nbytes / (kus * 1e-6) / 1e9, 1) if kus else None,
                             "frac": round(nbytes / (kus * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if kus else None}
            out.append(row)
    return out


def small_config(Q, name, steps=64, cpu_seconds=0.0):
    """Decode (exact and fast modes) and prefill of a smaller BASELINE config,
    and (cpu_seconds > 0) the CPU oracle's decode and prefill rates beside them."""
    cfg, base, tied, P = CONFIGS[name]
    m = Q.Model.synth(cfg, base, seed=1234, tied=tied)
    f = m.fork(Q.MODE_FAST)
    try:
        prompt = [int(t) for t in np.random.default_rng(1234).integers(0, cfg[0], P)]
        m.prefill(prompt, want_logits=True)
        m.reset(0)
        Q.lib().qllama_device_sync()
        t0 = time.perf_counter()
        m.prefill(prompt, want_logits=True)
        Q.lib().qllama_device_sync()
        t_pf = time.perf_counter() - t0
        res = {"cfg": cfg, "prefill_tokens": P, "prefill_tok_s": round(P / t_pf, 1)}
        n = min(steps, cfg[7] - P - 8)
        for cache, key in ((m, "exact"), (f, "fast")):
            if cache is f:
                f.prefill(prompt, want_logits=True)
            tok = int(np.argmax(cache.logits[0]))
            out = cache.generate_greedy(tok, 4)
            Q.lib().qllama_device_sync()
            pos = cache.pos
            t0 = time.perf_counter()
            cache.generate_greedy(out[-1], n)
            Q.lib().qllama_device_sync()
            t = time.perf_counter() - t0
            b = statistics.mean(decode_bytes(cfg, pos + 1 + i) for i in range(n))
            res[f"decode_{key}_tok_s"] = round(n / t, 1)
            res[f"decode_{key}_hbm_roofline_frac"] = round(b / (t / n) / (HBM_PEAK_GBS * 1e9), 4)
        res["decode_context"] = [P + 5, P + 4 + n]
        if cpu_seconds > 0:
            res["cpu_baseline"] = cpu_baseline(Q, m, cfg, base, P, cpu_seconds, prefill_tokens=P,
                                               prefill_seconds=cpu_seconds / 2)
        return res
    finally:
        f.close()
        m.close()


GPT2_SMALL = (50257, 768, 12, 12, 3072, 1024)   # vocab, d_model, heads, layers, d_ff, max_seq


def gpt2_decode(Q, prompt=32, steps=32):
    """GPT-2 (GPTC) KV decode at the GPT-2-small shape, fp32 (gpt_decode_step,
    host logits as in the reference): numpy N(0, 0.02) weights, gammas 1."""
    vocab, dm, nh, L, ff, S = GPT2_SMALL
    rng = np.random.default_rng(5)

    def w(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    one, zero = np.ones(dm, np.float32), np.zeros(dm, np.float32)
    t = [("wte", w(vocab, dm)), ("wpe", w(S, dm))]
    for _ in range(L):
        t += [("W_q", w(dm, dm)), ("W_k", w(dm, dm)), ("W_v", w(dm, dm)), ("W_o", w(dm, dm)),
              ("b_q", zero), ("b_k", zero), ("b_v", zero), ("b_o", zero), ("gamma1", one), ("beta1", zero),
              ("gamma2", one), ("beta2", zero), ("ff_W1", w(dm, ff)), ("ff_b1", np.zeros(ff, np.float32)),
              ("ff_W2", w(ff, dm)), ("ff_b2", zero)]
    t += [("ln_f_gamma", one), ("ln_f_beta", zero), ("lm_head", w(dm, vocab))]
    dec = Q.GPTDecoder(Q.host_gpt(GPT2_SMALL, t))
    try:
        ids = rng.integers(0, vocab, prompt)
        for tok in ids:
            lg = dec.step(int(tok))
        tok = int(np.argmax(lg))
        t0 = time.perf_counter()
        for _ in range(steps):
            tok = int(np.argmax(dec.step(tok)))
        dt = time.perf_counter() - t0
    finally:
        dec.close()
    wbytes = 4 * (L * (4 * dm * dm + 2 * dm * ff) + dm * vocab)
    kv = 4 * L * 2 * dm * (prompt + steps // 2)
    return {"shape": list(GPT2_SMALL), "dtype": "f32", "tok_s": round(steps / dt, 2),
            "ms_per_step": round(1e3 * dt / steps, 3), "context": [prompt + 1, prompt + steps],
            "hbm_roofline_frac": round((wbytes + kv) / (dt / steps) / (HBM_PEAK_GBS * 1e9), 4),
            "note": "gpt_decode_step with host logits each step (as model.c's callers use it)"}


def f32_host_model(Q, cfg, base, tied, seed=1234):
    """A reference LlamaModel (host f32) with N(0, 0.02) weights from numpy, norms 1,
    biases 0, in the canonical tensor order (llama.c:198-219)."""
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    rng = np.random.default_rng(seed)

    def w(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    one = np.ones(dm, np.float32)
    wte = w(vocab, dm)
    t = [("wte", wte)]
    for _ in range(L):
        t += [("attn_norm", one), ("Wq", w(dm, qd)), ("Wk", w(dm, kvd)), ("Wv", w(dm, kvd)),
              ("b_q", np.zeros(qd, np.float32)), ("b_k", np.zeros(kvd, np.float32)), ("b_v", np.zeros(kvd, np.float32)),
              ("Wo", w(qd, dm)), ("ffn_norm", one), ("Wgate", w(dm, ff)), ("Wup", w(dm, ff)), ("Wdown", w(ff, dm))]
    t += [("final_norm", one), ("lm_head", np.ascontiguousarray(wte.T) if tied else w(dm, vocab))]
    return Q.host_model(cfg, base, 1e-5, t)


def f32_bytes(cfg, t):
    """HBM bytes of one fp32 decode token at context t: every weight once (f32),
    the KV rows read and the new row written."""
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    w = L * (dm * (qd + 2 * kvd) + qd * dm + 2 * dm * ff + ff * dm) + dm * vocab
    return 4 * w + L * (2 * kvd * 4 * t + 2 * kvd * 4)


def main_f32(args, Q, cfg, base, tied, P):
    """The fp32 (LLMA) decode path: llama_decode_step per token (host logits, as in
    the reference), after P prompt tokens fed the same way."""
    W, K, NP = args.warmup, args.steps, args.profile_steps
    if P + W + K + NP > cfg[7]:
        sys.exit("bench.py: prompt + warmup + steps + profile exceeds max_seq")
    t0 = time.perf_counter()
    host = f32_host_model(Q, cfg, base, tied)
    t_host = time.perf_counter() - t0
    t0 = time.perf_counter()
    m = Q.FModel(host)                                   # uploads the weights
    t_up = time.perf_counter() - t0
    ids = list(np.random.default_rng(1234).integers(0, cfg[0], P + 1))
    for t in ids[:P]:
        lg = m.step(int(t))
    tok = int(np.argmax(lg)) if P else int(ids[P])
    for _ in range(W):
        tok = int(np.argmax(m.step(tok)))
    pos0 = m.pos
    t0 = time.perf_counter()
    for _ in range(K):
        tok = int(np.argmax(m.step(tok)))
    t_dec = time.perf_counter() - t0
    prof = {}
    if NP:
        Q.profile(True)
        for _ in range(NP):
            tok = int(np.argmax(m.step(tok)))
        prof = Q.profile_read()
        Q.profile(False)
    fwd = None
    FR = args.forward_rows
    if FR:
        # llama_model_forward (llama.c:167-186): FR rows through the batched
        # GEMMs and prefill attention, host logits (FR, vocab) as in the reference
        fids = [int(t) for t in np.random.default_rng(7).integers(0, cfg[0], FR)]
        m.forward(fids)                                  # first call: buffers, kernel loads
        t0 = time.perf_counter()
        m.forward(fids)
        t_fwd = time.perf_counter() - t0
        Q.profile(True)
        m.forward(fids)
        fprof = Q.profile_read()
        Q.profile(False)
        fwd = f32_forward_line(cfg, FR, t_fwd, fprof)
    m.close()
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    gb = {"gemv_qkv": (L, 4 * dm * (qd + 2 * kvd)), "gemv_o": (L, 4 * qd * dm), "gemv_gate_up": (L, 8 * dm * ff),
          "gemv_down": (L, 4 * ff * dm), "gemv_head": (1, 4 * dm * vocab)}
    gemv_ms = sum(prof[k][0] * n for k, (n, _) in gb.items() if k in prof)
    gemv_bytes = sum(n * b for n, b in gb.values())
    step_bytes = statistics.mean(f32_bytes(cfg, pos0 + 1 + i) for i in range(K))
    achieved = gemv_bytes / (gemv_ms * 1e-3) / 1e9 if gemv_ms else None
    line = {
        "metric": f"fp32 LLMA decode tok/s, {args.config}-shape (1 GPU)",
        "value": round(K / t_dec, 3), "unit": "tok/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(1e3 * t_dec / K, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (numpy N(0,0.02) f32 weights; uniform-random prompt ids)",
        "config": {"workload": f"{args.config}-shape fp32 LLaMA greedy decode (llama_decode_step, host logits) "
                               f"after {P} prompt tokens", "cfg": cfg, "context_timed": [pos0 + 1, pos0 + K]},
        "decode_hbm_roofline_frac": round(step_bytes / (t_dec / K) / (HBM_PEAK_GBS * 1e9), 4),
        "decode_bytes_per_token": int(step_bytes),
        "roofline": {"bound": "hbm", "kernel": "k_gemv_f32 (f32 GEMV, k-order chains, all call sites)",
                     "achieved": round(achieved, 1) if achieved else None, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None},
        "kernel_ms_per_token": {k: round(v[0] * v[1] / NP, 4) for k, v in sorted(prof.items())} if NP else None,
        "host_model_s": round(t_host, 2), "upload_s": round(t_up, 3),
        "forward": fwd,
    }
    print(json.dumps(line), flush=True)


def f32_forward_line(cfg, rows, t_s, prof):
    """The batched fp32 forward's rate and its GEMMs against the VALU bound: each
    multiply-add is a separate v_mul_f32 and v_add_f32 (the reference rounds every
    product before its add), so the ceiling is the unpacked, unfused fp32 lane rate."""
    vocab, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd
    macs = rows * (L * (dm * (qd + 2 * kvd) + qd * dm + 2 * dm * ff + ff * dm) + dm * vocab)
    ms = {k: v[0] * v[1] for k, v in prof.items()}
    gemm_ms = ms.get("pf_gemm", 0.0)
    tf = 2 * macs / (gemm_ms * 1e-3) / 1e12 if gemm_ms else None
    return {"rows": rows, "tok_s": round(rows / t_s, 1), "ms": round(1e3 * t_s, 3),
            "note": "llama_model_forward, host logits (rows, vocab) copied back inside the timed call",
            "kernel_ms": {k: round(v, 3) for k, v in sorted(ms.items())},
            "gemm": {"bound": "valu", "achieved": round(tf, 2) if tf else None,
                     "peak": F32_VALU_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tf / F32_VALU_TFLOPS, 4) if tf else None,
                     "peak_note": "unpacked fp32 v_mul + v_add, 256 CUs x 128 lanes x 2.4 GHz (a wave64 op "
                                  "every 2 cycles per SIMD; the product is rounded before its add, as in "
                                  "matrix.c:188, so no FMA or packed math); the published fp32 peak, "
                                  f"{F32_MFMA_TFLOPS} TFLOP/s, counts an FMA as two"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="8b", choices=sorted(CONFIGS))
    ap.add_argument("--prefill", type=int, default=None)
    ap.add_argument("--profile-steps", type=int, default=4)
    ap.add_argument("--sampled-steps", type=int, default=32,
                    help="decode steps with on-device sampling (T 0.8, top-k 40, top-p 0.95: the llama "
                         "command's settings), timed after the greedy ones")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="also run one plain device copy of this many MiB (the scale reference "
                         "for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--load-check", action="store_true",
                    help="also time q_llama_model_save and q_llama_model_load of the model through $TMPDIR "
                         "(writes a checkpoint of the model's size there)")
    ap.add_argument("--full-range", action=argparse.BooleanOptionalAction, default=True,
                    help="also decode from the prompt to max_seq in one loop per mode (the config's whole "
                         "decode range)")
    ap.add_argument("--extras", action=argparse.BooleanOptionalAction, default=True,
                    help="also measure the op-level GEMV / GQA configs, the 1B and tiny configs, the "
                         "PCIe-inclusive q_llama_decode_step rate and the GPT-2 decode")
    ap.add_argument("--forward-rows", type=int, default=512,
                    help="f32 path: also time llama_model_forward over this many rows (0: skip)")
    ap.add_argument("--path", default="int8", choices=["int8", "f32"],
                    help="int8: the headline LLMQ decode (default); f32: the LLMA decode path")
    ap.add_argument("--ops-only", action="store_true",
                    help="measure only the op-level GEMV and GQA configs (BASELINE configs 2-3) and print "
                         "them as the one JSON line (no model is built)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is a design note only)", file=sys.stderr)
        sys.exit(1)
    rank = int(os.environ.get("RANK", "0"))

    Q = load_qllama()
    if args.ops_only:
        line = {"metric": "op-level int8 GEMV and GQA decode attention (HBM roofline fraction)", "n_gpus": 1,
                "higher_is_better": True, "data": "synthetic", "op_gemv": op_gemv(Q), "op_gqa": op_gqa(Q)}
        if rank == 0:
            print(json.dumps(line), flush=True)
        return
    cfg, base, tied, prefill = CONFIGS[args.config]
    P = args.prefill if args.prefill is not None else prefill
    if args.path == "f32":
        return main_f32(args, Q, cfg, base, tied, args.prefill if args.prefill is not None else 64)
    W, K, NP, NS = args.warmup, args.steps, args.profile_steps, args.sampled_steps
    if P + W + K + 2 * NP + NS + (2 if NS else 0) > cfg[7]:
        sys.exit(f"bench.py: prefill {P} + warmup {W} + steps {K} + profile {NP} + sampled {NS} "
                 f"exceeds max_seq {cfg[7]}")

    t0 = time.perf_counter()
    gm = Q.Model.synth(cfg, base, seed=1234, tied=tied)
    t_build = time.perf_counter() - t0
    prompt = [int(t) for t in np.random.default_rng(1234).integers(0, cfg[0], P)]

    # prefill (timed separately, after one untimed ingestion of the same call: it
    # allocates the buffers and loads every kernel the call uses, logits path included)
    if P:
        gm.prefill(prompt, want_logits=True)
        gm.reset(0)
    Q.lib().qllama_device_sync()
    t0 = time.perf_counter()
    gm.prefill(prompt, want_logits=True)
    Q.lib().qllama_device_sync()
    t_prefill = time.perf_counter() - t0
    first = int(np.argmax(gm.logits[0]))

    def timed_decode(m, tok):
        """W untimed warm-up steps, then exactly K timed greedy steps on the device."""
        out = m.generate_greedy(tok, W) if W else []
        tok = out[-1] if out else tok
        Q.lib().qllama_device_sync()
        pos = m.pos
        t0 = time.perf_counter()
        out = m.generate_greedy(tok, K)
        Q.lib().qllama_device_sync()
        return time.perf_counter() - t0, pos, out[-1]

    def full_range(m):
        """From the prompt to max_seq in one device loop (the config's whole decode
        range: 512 steps at contexts 2049..2560 for the 8B shape)."""
        n = cfg[7] - P
        if n < 2:
            return None
        m.reset(0)
        m.prefill(prompt, want_logits=True)
        tok = int(np.argmax(m.logits[0]))
        Q.lib().qllama_device_sync()
        t0 = time.perf_counter()
        m.generate_greedy(tok, n)
        Q.lib().qllama_device_sync()
        t = time.perf_counter() - t0
        bytes_avg = statistics.mean(decode_bytes(cfg, P + 1 + i) for i in range(n))
        return {"tok_s": round(n / t, 3), "steps": n, "context": [P + 1, P + n],
                "ms_per_step": round(1e3 * t / n, 4),
                "hbm_roofline_frac": round(bytes_avg / (t / n) / (HBM_PEAK_GBS * 1e9), 4)}

    def kernel_profile(m, tok):
        if not NP:
            return {}
        Q.profile(True)
        m.generate_greedy(tok, NP)
        prof = Q.profile_read()
        Q.profile(False)
        return prof

    # exact mode (logits bit-identical to the reference; the headline), on the prefilled cache
    t_decode, pos_first, tok = timed_decode(gm, first)
    prof = kernel_profile(gm, tok)
    # fast mode (split-K attention, tree-ordered norm sums; greedy streams depart
    # from the reference's, see the design notes): a second cache on the same weights
    # On a fast cache the prompt's attention is the fp32 MFMA kernel with an online
    # softmax (not bit-exact either); timed after one untimed ingestion.
    gf = gm.fork(Q.MODE_FAST)
    t_prefill_fast = None
    if P:
        gf.prefill(prompt, want_logits=True)
        gf.reset(0)
        Q.lib().qllama_device_sync()
        t0 = time.perf_counter()
    gf.prefill(prompt, want_logits=True)
    Q.lib().qllama_device_sync()
    if P:
        t_prefill_fast = time.perf_counter() - t0
    t_fast, pos_fast, tok_f = timed_decode(gf, int(np.argmax(gf.logits[0])))
    assert pos_fast == pos_first
    prof_fast = kernel_profile(gf, tok_f)
    pf_fast_ms = None
    if P >= 16 and NP:
        gf.reset(0)
        Q.profile(True)
        gf.prefill(prompt, want_logits=False)
        pp = Q.profile_read()
        Q.profile(False)
        pf_fast_ms = {k: round(pp[k][0] * pp[k][1], 3) for k in ("pf_gemm", "pf_attn") if k in pp}
    ms_per_step = 1e3 * t_decode / K
    tok_s = K / t_decode
    # context of each timed step: pos + 1 cached rows
    ctx = [pos_first + 1 + i for i in range(K)]
    step_bytes = statistics.mean(decode_bytes(cfg, t) for t in ctx)
    step_frac = step_bytes / (t_decode / K) / (HBM_PEAK_GBS * 1e9)
    fast_line = {"tok_s": round(K / t_fast, 3), "ms_per_step": round(1e3 * t_fast / K, 4),
                 "hbm_roofline_frac": round(step_bytes / (t_fast / K) / (HBM_PEAK_GBS * 1e9), 4),
                 "parity": "not bit-exact; greedy stream departs from the reference (tests/test_gpu_fast.py)",
                 "kernel_ms_per_token": {k: round(v[0] * v[1] / NP, 4) for k, v in sorted(prof_fast.items())}
                 if NP else None,
                 "prefill_tok_s": round(P / t_prefill_fast, 2) if t_prefill_fast else None,
                 "prefill_kernel_ms": pf_fast_ms,
                 "prefill_attention": "fp32 MFMA, online softmax (k_pf_fa); the GEMMs are the exact int8 ones"}
    full = {"fast": full_range(gf), "exact": full_range(gm)} if args.full_range else None
    # sampled decode (sample_token's arithmetic on the device between the steps)
    sampled = None
    if NS:
        gm.reset(pos_first + K + NP)
        rng = Q.rng_create(1234)
        gm.generate(2, 0.8, 40, 0.95, rng)          # allocates the sampler's buffers
        Q.lib().qllama_device_sync()
        t0 = time.perf_counter()
        gm.generate(NS, 0.8, 40, 0.95, rng)
        Q.lib().qllama_device_sync()
        t_s = time.perf_counter() - t0
        sampled = {"tok_s": round(NS / t_s, 3), "steps": NS, "temperature": 0.8, "top_k": 40, "top_p": 0.95,
                   "ms_per_step": round(1e3 * t_s / NS, 4), "mode": "exact"}
    gf.close()
    # the drop-in q_llama_decode_step: logits copied to the host every token (PCIe),
    # argmax on the host, as the reference's loop does (main.c:663-668)
    step_host = None
    if args.extras and K:
        gm.reset(pos_first)
        n = min(K, 32)
        lg = gm.step(tok)
        t0 = time.perf_counter()
        for _ in range(n):
            lg = gm.step(int(np.argmax(lg)))
        t_h = time.perf_counter() - t0
        step_host = {"tok_s": round(n / t_h, 3), "steps": n, "ms_per_step": round(1e3 * t_h / n, 4),
                     "context": [pos_first + 2, pos_first + 1 + n]}
    extras = {}
    if args.extras and args.config == "8b":
        extras["op_gemv"] = op_gemv(Q)
        extras["op_gqa"] = op_gqa(Q)
        cs = 0.0 if args.no_cpu_baseline else args.cpu_seconds / 3
        extras["config_1b"] = small_config(Q, "1b", cpu_seconds=cs)
        extras["config_tiny"] = small_config(Q, "tiny", cpu_seconds=cs)
        extras["gpt2_decode"] = gpt2_decode(Q)
    if args.calib_copy_mib:
        Q.lib().qllama_test_copy.argtypes = [C.c_size_t]
        if Q.lib().qllama_test_copy(args.calib_copy_mib << 20) != 0:
            raise RuntimeError("calibration copy failed")
    gb = gemv_bytes(cfg)
    # the GEMV sites that run as kernels of their own (the QKV GEMV runs inside the
    # attention-half launch on the shapes that launch serves): bytes and times of
    # the same sites
    gb = {k: v for k, v in gb.items() if k in prof}
    gemv_ms = sum(prof[k][0] * n for k, (n, _) in gb.items())
    gemv_bytes_tok = sum(n * b for (n, b) in gb.values())
    launches_per_tok = sum(n for (n, _) in gb.values())
    achieved = gemv_bytes_tok / (gemv_ms * 1e-3) / 1e9 if gemv_ms > 0 else None
    traffic = None
    if args.config == "8b" and os.path.exists(TRAFFIC_JSON):
        per = json.load(open(TRAFFIC_JSON))["bytes_per_dispatch"]
        if gb and all(k in per for k in gb):
            traffic = round(sum(n * per[k] for k, (n, _) in gb.items()) / launches_per_tok)

    # prefill GEMMs on MFMA: a second, profiled ingestion of the same prompt
    pf_roof = None
    if P >= 16 and NP:
        gm.reset(0)
        Q.profile(True)
        gm.prefill(prompt, want_logits=False)
        pprof = Q.profile_read()
        Q.profile(False)
        if "pf_gemm" in pprof:
            g_ms = pprof["pf_gemm"][0] * pprof["pf_gemm"][1]
            a_ms = pprof["pf_attn"][0] * pprof["pf_attn"][1] if "pf_attn" in pprof else None
            tops = prefill_gemm_ops(cfg, P) / (g_ms * 1e-3) / 1e12
            pf_roof = {"bound": "mfma", "kernel": "k_gemm_i8 (int8 MFMA GEMM, all call sites)",
                       "achieved": round(tops, 1), "peak": INT8_MFMA_PEAK_TOPS, "unit": "TOP/s",
                       "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4), "gemm_ms": round(g_ms, 3),
                       "attention_ms": round(a_ms, 3) if a_ms is not None else None}

    load = None
    if args.load_check:
        import tempfile
        d = tempfile.mkdtemp(dir=os.environ.get("TMPDIR"))
        path = os.path.join(d, "model.llmq")
        h = gm.hash()
        t0 = time.perf_counter()
        gm.save(path)
        t_save = time.perf_counter() - t0
        size = os.path.getsize(path)
        times = []
        for _ in range(2):                       # the second read finds the file in the page cache
            t0 = time.perf_counter()
            m2 = Q.Model.load(path)
            times.append(time.perf_counter() - t0)
            ok = m2.hash() == h
            m2.close()
            if not ok:
                raise RuntimeError("loaded weights differ from the saved model")
        os.remove(path)
        os.rmdir(d)
        load = {"bytes": size, "save_s": round(t_save, 3), "load_s": [round(t, 3) for t in times],
                "load_gbs": [round(size / t / 1e9, 2) for t in times]}
    cpu = None
    if not args.no_cpu_baseline and rank == 0:
        cpu = cpu_baseline(Q, gm, cfg, base, pos_first, args.cpu_seconds, prefill_tokens=P,
                           prefill_seconds=args.cpu_seconds / 2)
    gm.close()

    line = {
        "metric": METRIC,
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded N(0,0.02) weights quantized per channel; uniform-random prompt ids)",
        "config": {
            "workload": f"{args.config}-shape int8 LLaMA greedy decode after a {P}-token prefill",
            "cfg": cfg, "rope_base": base, "tied": tied, "prefill_tokens": P,
            "context_timed": [ctx[0], ctx[-1]], "decode_mode": "exact",
        },
        "decode_hbm_roofline_frac": round(step_frac, 4),
        "decode_fast": fast_line,
        "decode_step_host_logits": step_host,
        "decode_full_range": full,
        "decode_bytes_per_token": int(step_bytes),
        "prefill_tok_s": round(P / t_prefill, 2) if P else None,
        "sampled_decode": sampled,
        "checkpoint_io": load,
        "prefill_roofline": pf_roof,
        "prefill_s": round(t_prefill, 4),
        "model_build_s": round(t_build, 3),
        "roofline": {
            "bound": "hbm",
            "kernel": "W8A8 int8 decode GEMV (k_gemv_ws / k_gemv_dec), every site launched on its own: "
                      + ", ".join(sorted(gb)),
            "achieved": round(achieved, 1) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": traffic,
            "bytes_per_launch": round(gemv_bytes_tok / launches_per_tok) if launches_per_tok else None,
            "avg_launch_us": round(1e3 * gemv_ms / launches_per_tok, 3) if gemv_ms else None,
        },
        "kernel_ms_per_token": {k: round(v[0] * v[1] / NP, 4) for k, v in sorted(prof.items())} if NP else None,
        "cpu_baseline": cpu,
    }
    line.update(extras)
    if rank == 0:
        print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
