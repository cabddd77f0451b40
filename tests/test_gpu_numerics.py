"""GPU numerics: the device's exact evaluation of a sequential float32 sum of
non-negative terms (used for rmsnorm's sum of squares, rmsnorm.c:15, and the
softmax denominator, llama.c:567) must equal the plain left-to-right float32
loop bit for bit on every input.  The loop is numpy's add.accumulate over
float32, which adds strictly in order."""
import ctypes as C

import numpy as np
import pytest

import qlib

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    lib = qlib.load().lib()
    lib.qllama_test_seqsum.argtypes = [C.POINTER(C.c_float), C.c_int, C.POINTER(C.c_float), C.POINTER(C.c_int)]
    return lib


def seq_ref(a):
    a = np.ascontiguousarray(a, np.float32)
    if a.size == 0:
        return np.float32(0.0)
    return np.add.accumulate(a, dtype=np.float32)[-1]


def dev_sum(L, a):
    a = np.ascontiguousarray(a, np.float32)
    out = C.c_float()
    info = (C.c_int * 2)()
    rc = L.qllama_test_seqsum(a.ctypes.data_as(C.POINTER(C.c_float)), a.size, C.byref(out), info)
    assert rc == 0
    return np.float32(out.value), info[0], info[1]


def cases():
    rng = np.random.default_rng(12345)
    out = []
    for n in (0, 1, 2, 3, 7, 64, 288, 1023, 1024, 1025, 2048, 2300, 4096, 8192, 14336, 16384):
        out.append(("squares", (rng.standard_normal(n).astype(np.float32)) ** 2))
    for n in (1, 129, 2049, 2560, 8192):
        for sig in (0.05, 1.0, 4.0, 12.0, 40.0):
            s = (rng.standard_normal(n) * sig).astype(np.float32)
            out.append((f"softmax{sig}", np.exp(s - s.max()).astype(np.float32)))
    for n in (100, 4096):
        out.append(("ties", (rng.integers(0, 64, n) * np.float32(2.0 ** -6)).astype(np.float32)))
        out.append(("halves", np.full(n, 0.5, np.float32)))
        out.append(("ones", np.ones(n, np.float32)))
        out.append(("pow2", np.exp2(rng.integers(-30, 30, n)).astype(np.float32)))
        out.append(("wide", np.exp2(rng.uniform(-120, 120, n)).astype(np.float32)))
        out.append(("subnormal", (rng.integers(0, 1000, n) * np.float32(2.0 ** -149)).astype(np.float32)))
        z = (rng.standard_normal(n) ** 2).astype(np.float32)
        z[rng.random(n) < 0.5] = 0
        out.append(("zeros", z))
        out.append(("growing", np.arange(n, dtype=np.float32) * np.float32(1.5)))
        out.append(("one_big", np.concatenate([[np.float32(3e8)], np.full(n - 1, 1.0, np.float32)])))
        out.append(("big_last", np.concatenate([np.full(n - 1, 1e-3, np.float32), [np.float32(7e5)]])))
        # a sum parked on 1.0 whose later terms fall just below / at / above half an ulp
        half = np.float32(2.0 ** -24)
        for tail in (np.nextafter(half, np.float32(0)), half, np.nextafter(half, np.float32(1))):
            out.append(("absorbed", np.concatenate([[np.float32(1.0)], np.full(n - 1, tail, np.float32)])))
        out.append(("edge_mix", np.concatenate([[np.float32(1.0)],
                                                (rng.integers(0, 4, n - 1) * half).astype(np.float32)])))
    return out


def test_sequential_sum_is_exact(L):
    fallbacks, total_hard, bad = 0, 0, []
    for name, a in cases():
        got, nhard, fell = dev_sum(L, a)
        want = seq_ref(a)
        if got.view(np.uint32) != np.float32(want).view(np.uint32):
            bad.append((name, a.size, float(got), float(want)))
        fallbacks += fell
        total_hard += nhard
    assert not bad, bad[:5]
    print(f"seqsum: {len(cases())} cases exact; fallbacks={fallbacks}; hard steps={total_hard}")


def test_sequential_sum_random_sweep(L):
    rng = np.random.default_rng(7)
    bad = 0
    fb = 0
    for trial in range(300):
        n = int(rng.integers(1, 16385))
        kind = trial % 3
        if kind == 0:
            a = (rng.standard_normal(n).astype(np.float32) * np.float32(rng.uniform(0.01, 100))) ** 2
        elif kind == 1:
            s = (rng.standard_normal(n) * rng.uniform(0.1, 20)).astype(np.float32)
            a = np.exp(s - s.max()).astype(np.float32)
        else:
            a = np.abs(rng.standard_cauchy(n)).astype(np.float32)
        got, _, fell = dev_sum(L, a)
        bad += got.view(np.uint32) != seq_ref(a).view(np.uint32)
        fb += fell
    assert bad == 0
    # the fast path must be the common case on model-like data
    assert fb <= 10, f"{fb} of 300 sums fell back to the serial loop"
