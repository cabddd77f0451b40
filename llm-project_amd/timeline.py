#!/usr/bin/env python3
"""Per-block timeline of one decode layer, from the stamps of libqllama_tl.so.

Build the stamped library first (`make -C llm-project_amd timeline`; the stamps
of qdev_tl.h are compiled out of libqllama.so).  This script builds a model of
the given shape from the seeded generator, ingests a prompt, runs greedy decode
steps (HIP-graph replays, as the bench does) and prints, for the last layer of
the last step:

* one row per kernel: first block start and last block end relative to the
  layer's first kernel, the kernel's span, and the gap to the previous kernel;
* the phases inside the kernels: for the GEMVs with a prologue, when the
  quantized activation is ready and when the first row is done; for the decode
  attention, when the scores' K tile is loaded, and in the PV blocks when the
  block maxima, the exact softmax sum and the weights are in, and when the
  chains end (median and max over blocks, from each block's own start).

Clock: the device's constant 100 MHz counter, so stamps are 10 ns apart at best.

  python3 llm-project_amd/timeline.py [--config 8b] [--steps 4] [--json OUT]
"""
import argparse
import ctypes as C
import importlib.util
import json
import os
import statistics
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
KERNELS, BLOCKS, EVENTS = 8, 1024, 8
TICK_US = 0.01

CONFIGS = {
    # vocab, d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq; rope base; tied; prefill
    "8b": ([128256, 4096, 32, 32, 8, 128, 14336, 2560], 500000.0, False, 2048),
    "1b": ([128256, 2048, 16, 32, 8, 64, 8192, 768], 500000.0, True, 512),
    "tiny": ([32000, 288, 6, 6, 2, 48, 768, 256], 10000.0, False, 128),
}

# (unit, kernel id) -> name, in the order the layer runs them; events per kernel
LAYER = [
    (("gemv", 0), "gemv_qkv (k_gemv_ws, rmsnorm prologue)", {1: "prologue done", 2: "row waves see x", 3: "first row done"}),
    (("attn", 3), "attn_layer Q phase (QKV rows of one KV head)",
     {6: "x arrived", 1: "prologue done", 2: "first row (weights in)", 3: "rows stored", 5: "at the meeting"}),
    (("attn", 0), "attn_scores (k_attn_scores; S phase of k_attn_layer)", {1: "K tile + q in LDS"}),
    (("attn", 1), "attn_pv (k_attn_pv; P phase of k_attn_layer)", {1: "block maxima", 2: "exact sum", 3: "weights in LDS", 5: "chains end"}),
    (("gemv", 1), "gemv_o (k_gemv_ws, quantizes o)", {1: "prologue done", 2: "row waves see x", 3: "first row done"}),
    (("gemv", 2), "gemv_gate_up (k_gemv_ws, rmsnorm prologue)", {1: "prologue done", 2: "row waves see x", 3: "first row done"}),
    (("gemv", 7), "quant_h (k_quant_blocks)", {}),
    (("gemv", 4), "gemv_down (k_gemv_dec)", {}),
    (("gemv", 5), "gemv_down (k_gemv_ws, quantizes h)", {1: "prologue done", 2: "row waves see x", 3: "first row done"}),
]


def load_qllama(lib_path):
    spec = importlib.util.spec_from_file_location("qllama", os.path.join(HERE, "qllama.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    mod.LIB_PATH = lib_path
    return mod


def read(L, unit):
    buf = (C.c_ulonglong * (KERNELS * BLOCKS * EVENTS))()
    fn = getattr(L, f"qllama_tl_read_{unit}")
    fn.argtypes = [C.c_void_p, C.c_int]
    if fn(C.cast(buf, C.c_void_p), 0) != 0:
        raise RuntimeError(f"qllama_tl_read_{unit} failed")
    return np.frombuffer(buf, dtype=np.uint64).reshape(KERNELS, BLOCKS, EVENTS).astype(np.int64)


def kernel_blocks(a, kid):
    """Stamps of the blocks that ran (event 0 set) of one kernel id."""
    k = a[kid]
    return k[k[:, 0] > 0]


def summarize(bufs, spec):
    rows, t0, prev_end = [], None, None
    for (unit, kid), name, evs in spec:
        b = kernel_blocks(bufs[unit], kid)
        if not len(b):
            rows.append({"kernel": name, "blocks": 0})
            continue
        start, end = int(b[:, 0].min()), int(b[:, 4].max())
        if t0 is None:
            t0 = start
        r = {"kernel": name, "blocks": int(len(b)), "start_us": round((start - t0) * TICK_US, 2),
             "end_us": round((end - t0) * TICK_US, 2), "span_us": round((end - start) * TICK_US, 2),
             "gap_before_us": round((start - prev_end) * TICK_US, 2) if prev_end is not None else None,
             "block_start_spread_us": round((int(b[:, 0].max()) - start) * TICK_US, 2),
             "xccs": int(len(set(int(v) >> 16 for v in b[:, 7])))}
        phases = {}
        for ev, label in evs.items():
            ok = b[:, ev] > 0
            if not ok.any():
                continue
            rel = (b[ok, ev] - b[ok, 0]) * TICK_US
            absl = (b[ok, ev] - start) * TICK_US
            phases[label] = {"median_from_block_start_us": round(float(np.median(rel)), 2),
                             "max_from_kernel_start_us": round(float(absl.max()), 2)}
        dur = (b[:, 4] - b[:, 0]) * TICK_US
        phases["block end"] = {"median_from_block_start_us": round(float(np.median(dur)), 2),
                               "max_from_kernel_start_us": round((end - start) * TICK_US, 2)}
        r["phases"] = phases
        rows.append(r)
        prev_end = end
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="8b", choices=sorted(CONFIGS))
    ap.add_argument("--prefill", type=int, default=None)
    ap.add_argument("--steps", type=int, default=4)
    ap.add_argument("--json", default=None)
    ap.add_argument("--lib", default=os.path.join(HERE, "libqllama_tl.so"))
    a = ap.parse_args()
    Q = load_qllama(a.lib)
    L = Q.lib()
    if not hasattr(L, "qllama_tl_read_gemv"):
        sys.exit(f"{a.lib} has no timeline stamps: build it with `make -C llm-project_amd timeline`")
    cfg, base, tied, P = CONFIGS[a.config]
    P = a.prefill if a.prefill is not None else P
    m = Q.Model.synth(cfg, base, seed=1234, tied=tied)
    prompt = [int(t) for t in np.random.default_rng(1234).integers(0, cfg[0], P)]
    m.prefill(prompt, want_logits=True)
    tok = int(np.argmax(m.logits[0]))
    failed = None
    try:
        m.generate_greedy(tok, a.steps)
    except RuntimeError as e:       # the stamps still tell where the blocks ran
        failed = str(e)
    L.qllama_device_sync()
    bufs = {u: read(L, u) for u in ("gemv", "attn")}
    ly = bufs["attn"][3]
    ran = ly[:, 0] > 0
    if ran.any():
        nb = int(ran.sum())
        xcc = (ly[:nb, 7] >> 16) & 0xF
        off = [int(b) for b in range(nb) if int(xcc[b]) != b % 8]
        print(f"k_attn_layer: {nb} blocks; {len(off)} not on XCD block % 8"
              + (f" (block: XCD {', '.join(f'{b}: {int(xcc[b])}' for b in off[:24])})" if off else ""))
    if failed:
        sys.exit(f"timeline: {failed}")
    ctx = P + a.steps
    layer = summarize(bufs, LAYER)
    # the PV chain rate: shader-clock cycles (kernel id 2) and wall time (kernel id 1)
    # between barrier 0 and the chain's end, per position
    pv, cyc = bufs["attn"][1], bufs["attn"][2]
    ok = (pv[:, 0] > 0) & (cyc[:, 1] > cyc[:, 0]) & (pv[:, 5] > pv[:, 3])
    chain = None
    if ok.any():
        cpp = (cyc[ok, 1] - cyc[ok, 0]) / ctx
        npp = (pv[ok, 5] - pv[ok, 3]) * TICK_US * 1e3 / ctx
        chain = {"positions": ctx, "cycles_per_position_median": round(float(np.median(cpp)), 2),
                 "ns_per_position_median": round(float(np.median(npp)), 3),
                 "clock_ghz_median": round(float(np.median(cpp / npp)), 3)}
    m.close()
    print(f"# {a.config}: last layer of decode step {a.steps} (context {ctx})")
    print("| kernel | blocks | XCDs | start us | end us | span us | gap before us | block starts spread us |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|")
    for r in layer:
        if not r["blocks"]:
            print(f"| {r['kernel']} | 0 | | | | | | |")
            continue
        g = "" if r["gap_before_us"] is None else f"{r['gap_before_us']:.2f}"
        print(f"| {r['kernel']} | {r['blocks']} | {r['xccs']} | {r['start_us']:.2f} | {r['end_us']:.2f} | "
              f"{r['span_us']:.2f} | {g} | {r['block_start_spread_us']:.2f} |")
    print("\n| kernel | phase | median from its block's start us | latest from the kernel's start us |")
    print("|---|---|---:|---:|")
    for r in layer:
        for label, p in r.get("phases", {}).items():
            print(f"| {r['kernel']} | {label} | {p['median_from_block_start_us']:.2f} | "
                  f"{p['max_from_kernel_start_us']:.2f} |")
    # the Q prologue of k_attn_layer, wave 0 (kernel id 4): x arrival (event 0),
    # rmsnorm applied (1), quantized (2); shader cycles of rmsnorm_apply (3 -> 5)
    q = bufs["attn"][4]
    okq = (q[:, 0] > 0) & (q[:, 2] > q[:, 0]) & (q[:, 5] > q[:, 3])
    if okq.any():
        print(f"\nQ prologue (wave 0, median over blocks): rmsnorm applied "
              f"{float(np.median(q[okq, 1] - q[okq, 0])) * TICK_US:.2f} us after x arrived "
              f"({float(np.median(q[okq, 5] - q[okq, 3])):.0f} shader cycles), quantized "
              f"{float(np.median(q[okq, 2] - q[okq, 0])) * TICK_US:.2f} us after")
    if chain:
        print(f"\nPV chains: {chain['cycles_per_position_median']} shader cycles per position "
              f"({chain['ns_per_position_median']} ns at {chain['clock_ghz_median']} GHz; median over blocks, "
              f"weights in LDS to chain end, {ctx} positions)")
    if a.json:
        with open(a.json, "w") as f:
            json.dump({"config": a.config, "context": ctx, "layer": layer, "pv_chain": chain}, f,
                      indent=1)


if __name__ == "__main__":
    main()
