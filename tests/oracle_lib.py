"""ctypes bindings to oracle/liboracle*.so, the CPU checker (test infrastructure).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module.  The restatement it loads follows the reference file:line cited at each
function in oracle/oracle.c.
"""
import ctypes as C
import struct
import os
import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")


class OrQT(C.Structure):
    _fields_ = [("rows", C.c_int), ("cols", C.c_int),
                ("q", C.POINTER(C.c_int8)), ("scale", C.POINTER(C.c_float))]


class OrBlock(C.Structure):
    _fields_ = [("attn_norm", C.POINTER(C.c_float)), ("ffn_norm", C.POINTER(C.c_float)),
                ("b_q", C.POINTER(C.c_float)), ("b_k", C.POINTER(C.c_float)),
                ("b_v", C.POINTER(C.c_float)),
                ("Wq", OrQT), ("Wk", OrQT), ("Wv", OrQT), ("Wo", OrQT),
                ("Wgate", OrQT), ("Wup", OrQT), ("Wdown", OrQT)]


class OrModel(C.Structure):
    _fields_ = [("vocab", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int),
                ("n_heads", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("d_ff", C.c_int), ("max_seq", C.c_int),
                ("rope_base", C.c_float), ("eps", C.c_float),
                ("wte", OrQT), ("blocks", C.POINTER(OrBlock)),
                ("final_norm", C.POINTER(C.c_float)), ("lm_head", OrQT)]


class OrFBlock(C.Structure):
    _fields_ = [(n, C.POINTER(C.c_float)) for n in
                ("attn_norm", "ffn_norm", "b_q", "b_k", "b_v", "Wq", "Wk", "Wv", "Wo", "Wgate", "Wup", "Wdown")]


class OrFModel(C.Structure):
    _fields_ = [("vocab", C.c_int), ("d_model", C.c_int), ("n_layers", C.c_int),
                ("n_heads", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("d_ff", C.c_int), ("max_seq", C.c_int),
                ("rope_base", C.c_float), ("eps", C.c_float),
                ("wte", C.POINTER(C.c_float)), ("blocks", C.POINTER(OrFBlock)),
                ("final_norm", C.POINTER(C.c_float)), ("lm_head", C.POINTER(C.c_float))]


class OrGBlock(C.Structure):
    _fields_ = [(n, C.POINTER(C.c_float)) for n in
                ("Wq", "Wk", "Wv", "Wo", "bq", "bk", "bv", "bo", "g1", "be1", "g2", "be2", "W1", "bf1", "W2", "bf2")]


class OrGPT(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "d_model", "n_heads", "n_layers", "d_ff", "max_seq")] + \
               [("wte", C.POINTER(C.c_float)), ("wpe", C.POINTER(C.c_float)), ("blocks", C.POINTER(OrGBlock)),
                ("lnf_g", C.POINTER(C.c_float)), ("lnf_b", C.POINTER(C.c_float)), ("lm_head", C.POINTER(C.c_float))]


class OrKV(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("max_seq", C.c_int), ("kv_dim", C.c_int),
                ("len", C.c_int), ("k", C.POINTER(C.c_float)), ("v", C.POINTER(C.c_float))]


def _cpu_has_avx512():
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return all(x in flags for x in ("avx512f", "avx512bw", "avx512vl", "avx512dq"))
    except OSError:
        return False


_lib = None


def lib():
    global _lib
    if _lib is None:
        name = "liboracle_v4.so" if _cpu_has_avx512() else "liboracle.so"
        path = os.path.join(ORACLE_DIR, name)
        if not os.path.exists(path):
            path = os.path.join(ORACLE_DIR, "liboracle.so")
        L = C.CDLL(path)
        fp = C.POINTER(C.c_float)
        i8p = C.POINTER(C.c_int8)
        L.or_qmatmul_ex.argtypes = [fp, C.c_int, C.POINTER(OrQT), fp, i8p, fp, C.POINTER(C.c_int32)]
        L.or_quantize_int8_percol.argtypes = [fp, C.c_int, C.c_int, i8p, fp]
        L.or_dequantize_int8_percol.argtypes = [i8p, fp, C.c_int, C.c_int, fp]
        L.or_rmsnorm.argtypes = [fp, C.c_int, C.c_int, fp, C.c_float, fp]
        L.or_rope_heads_pos.argtypes = [fp, C.c_int, C.c_int, C.c_int, C.c_float, C.c_int]
        L.or_gqa_forward.argtypes = [fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, fp, fp]
        L.or_attn_decode.argtypes = [fp, fp, fp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, fp, fp]
        L.or_argmax.argtypes = [fp, C.c_int]
        L.or_argmax.restype = C.c_int
        L.or_model_synth.argtypes = [C.POINTER(OrModel), C.POINTER(C.c_int32), C.c_float, C.c_float,
                                     C.c_uint64, C.c_int]
        L.or_model_alloc.argtypes = [C.POINTER(OrModel), C.POINTER(C.c_int32), C.c_float, C.c_float]
        L.or_model_quantize_from.argtypes = [C.POINTER(OrModel), C.POINTER(OrFModel)]
        L.or_model_free.argtypes = [C.POINTER(OrModel)]
        L.or_model_hash.argtypes = [C.POINTER(OrModel)]
        L.or_model_hash.restype = C.c_uint64
        L.or_kv_create.argtypes = [C.POINTER(OrKV), C.POINTER(OrModel)]
        L.or_kv_free.argtypes = [C.POINTER(OrKV)]
        L.or_decode_step.argtypes = [C.POINTER(OrModel), C.POINTER(OrKV), C.c_int, fp]
        L.or_expf_mismatches.argtypes = [C.c_uint32, C.c_uint32, fp]
        L.or_expf_mismatches.restype = C.c_longlong
        L.or_set_threads.argtypes = [C.c_int]
        L.or_matmul_row.argtypes = [fp, fp, C.c_int, C.c_int, fp]
        L.or_fmodel_synth.argtypes = [C.POINTER(OrFModel), C.POINTER(C.c_int32), C.c_float, C.c_float,
                                      C.c_uint64, C.c_int]
        L.or_fmodel_free.argtypes = [C.POINTER(OrFModel)]
        L.or_fkv_create.argtypes = [C.POINTER(OrKV), C.POINTER(OrFModel)]
        L.or_f32_decode_step.argtypes = [C.POINTER(OrFModel), C.POINTER(OrKV), C.c_int, fp]
        L.or_layernorm.argtypes = [fp, C.c_int, C.c_int, fp, fp, C.c_float, fp]
        L.or_gelu.argtypes = [fp, C.c_size_t, fp]
        L.or_gpt_synth.argtypes = [C.POINTER(OrGPT), C.POINTER(C.c_int32), C.c_uint64]
        L.or_gpt_alloc.argtypes = [C.POINTER(OrGPT), C.POINTER(C.c_int32)]
        L.or_gpt_free.argtypes = [C.POINTER(OrGPT)]
        L.or_gpt_hash.argtypes = [C.POINTER(OrGPT)]
        L.or_gpt_hash.restype = C.c_uint64
        L.or_gkv_create.argtypes = [C.POINTER(OrKV), C.POINTER(OrGPT)]
        L.or_gpt_decode_step.argtypes = [C.POINTER(OrGPT), C.POINTER(OrKV), C.c_int, fp]
        L.or_tanhf_mismatches.argtypes = [C.c_uint32, C.c_uint32, fp]
        L.or_tanhf_mismatches.restype = C.c_longlong
        L.or_rng_create.argtypes = [C.c_uint64]
        L.or_rng_create.restype = C.c_uint64
        L.or_rng_uniform.argtypes = [C.POINTER(C.c_uint64)]
        L.or_rng_uniform.restype = C.c_float
        L.or_sample_token.argtypes = [fp, C.c_int, C.c_float, C.c_int, C.c_float, C.POINTER(C.c_uint64)]
        L.or_get_threads.restype = C.c_int
        L.syn_key.argtypes = [C.c_uint64, C.c_uint64]
        L.syn_key.restype = C.c_uint64
        L.syn_fill.argtypes = [fp, C.c_size_t, C.c_uint64, C.c_uint64, C.c_double]
        L.syn_prompt.argtypes = [C.POINTER(C.c_int), C.c_int, C.c_uint64, C.c_int]
        L.syn_hash_f32.argtypes = [fp, C.c_size_t, C.c_uint64]
        L.syn_hash_f32.restype = C.c_uint64
        L.syn_hash_i8.argtypes = [i8p, C.c_size_t, C.c_uint64]
        L.syn_hash_i8.restype = C.c_uint64
        L.syn_ln.argtypes = [C.c_double]
        L.syn_ln.restype = C.c_double
        L.syn_sqrt.argtypes = [C.c_double]
        L.syn_sqrt.restype = C.c_double
        L.syn_cos_sin_2pi.argtypes = [C.c_double, C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.syn_normal.argtypes = [C.c_uint64, C.c_uint64]
        L.syn_normal.restype = C.c_double
        _lib = L
    return _lib


def fptr(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def i8ptr(a):
    assert a.dtype == np.int8 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_int8))


# ---- thin numpy wrappers --------------------------------------------------
def synth(n, seed, tid, sigma):
    out = np.empty(n, np.float32)
    lib().syn_fill(fptr(out), n, seed, tid, sigma)
    return out


def prompt(n, seed, vocab):
    ids = (C.c_int * n)()
    lib().syn_prompt(ids, n, seed, vocab)
    return list(ids)


def qfrom_tensors(cfg, gain_sigma, bias_sigma, seed=21):
    """The fp32 model of the quantize_from fixtures (tests/golden/gen_golden.c
    run_qfrom), as (name, array) pairs in the canonical LLMA order
    (llama.c:198-219): generator weights N(0, 0.3), embeddings N(0, 1), gains
    1 + N(0, g) and biases N(0, b) (1 and 0 when the sigma is 0), lm_head's
    column 5 zero."""
    V, dm, L, H, KVH, hd, ff, _ = cfg
    qd, kvd = H * hd, KVH * hd

    def fill(shape, tid, sigma, base=0.0):
        n = int(np.prod(shape))
        if sigma <= 0:
            return np.full(shape, base, np.float32)
        # the fixture generator keeps sigma as a float32 (0.1f) and widens it
        return (np.float32(base) + synth(n, seed, tid, float(np.float32(sigma)))).reshape(shape).astype(np.float32)

    out = [("wte", synth(V * dm, seed, 0, 1.0).reshape(V, dm))]
    for l in range(L):
        t0, u = 1 + 12 * l, 1000 + 8 * l
        out += [("attn_norm", fill((dm,), u, gain_sigma, 1.0)),
                ("Wq", synth(dm * qd, seed, t0 + 1, 0.3).reshape(dm, qd)),
                ("Wk", synth(dm * kvd, seed, t0 + 2, 0.3).reshape(dm, kvd)),
                ("Wv", synth(dm * kvd, seed, t0 + 3, 0.3).reshape(dm, kvd)),
                ("b_q", fill((qd,), u + 1, bias_sigma)), ("b_k", fill((kvd,), u + 2, bias_sigma)),
                ("b_v", fill((kvd,), u + 3, bias_sigma)),
                ("Wo", synth(qd * dm, seed, t0 + 7, 0.3).reshape(qd, dm)),
                ("ffn_norm", fill((dm,), u + 4, gain_sigma, 1.0)),
                ("Wgate", synth(dm * ff, seed, t0 + 9, 0.3).reshape(dm, ff)),
                ("Wup", synth(dm * ff, seed, t0 + 10, 0.3).reshape(dm, ff)),
                ("Wdown", synth(ff * dm, seed, t0 + 11, 0.3).reshape(ff, dm))]
    head = synth(dm * V, seed, 2 + 12 * L, 0.3).reshape(dm, V)
    head[:, 5] = 0.0
    return out + [("final_norm", fill((dm,), 999, gain_sigma, 1.0)), ("lm_head", head)]


def tensors_hash(tensors):
    """The fixtures' fp32 digest: h = h*31 + hash of each tensor, canonical order."""
    h = 0
    for i, (_, t) in enumerate(tensors):
        d = hash_f32(t)
        h = d if i == 0 else (h * 31 + d) & 0xFFFFFFFFFFFFFFFF
    return h


def hash_f32(a):
    a = np.ascontiguousarray(a, np.float32)
    return int(lib().syn_hash_f32(fptr(a), a.size, 0))


def hash_i8(a):
    a = np.ascontiguousarray(a, np.int8)
    return int(lib().syn_hash_i8(i8ptr(a), a.size, 0))


def quantize(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.int8)
    s = np.empty(cols, np.float32)
    lib().or_quantize_int8_percol(fptr(w), rows, cols, i8ptr(q), fptr(s))
    return q, s


def dequantize(q, s):
    rows, cols = q.shape
    w = np.empty((rows, cols), np.float32)
    lib().or_dequantize_int8_percol(i8ptr(np.ascontiguousarray(q)), fptr(np.ascontiguousarray(s)),
                                    rows, cols, fptr(w))
    return w


def qmatmul(A, q, s, intermediates=False):
    """C = qmatmul(A, W) with W given as int8 (K, N) + scales (N) (quant.c:60-85)."""
    A = np.ascontiguousarray(A, np.float32)
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s, np.float32)
    M, K = A.shape
    N = q.shape[1]
    W = OrQT(K, N, i8ptr(q), fptr(s))
    Cm = np.empty((M, N), np.float32)
    if not intermediates:
        lib().or_qmatmul_ex(fptr(A), M, C.byref(W), fptr(Cm), None, None, None)
        return Cm
    qa = np.empty((M, K), np.int8)
    as_ = np.empty(M, np.float32)
    acc = np.empty((M, N), np.int32)
    lib().or_qmatmul_ex(fptr(A), M, C.byref(W), fptr(Cm), i8ptr(qa), fptr(as_),
                        acc.ctypes.data_as(C.POINTER(C.c_int32)))
    return Cm, qa, as_, acc


def rmsnorm(x, g, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().or_rmsnorm(fptr(x), rows, cols, fptr(np.ascontiguousarray(g, np.float32)), eps, fptr(y))
    return y


def rope(x, n_heads, base, pos0):
    x = np.array(x, np.float32, copy=True, order="C")
    rows, cols = x.shape
    lib().or_rope_heads_pos(fptr(x), rows, cols, n_heads, base, pos0)
    return x


def attn_decode(q, kc, vc, pos, n_heads, n_kv, hd):
    """llama.c:554-576 over cache rows 0..pos; kc/vc are [>=pos+1, n_kv*hd]."""
    kc = np.ascontiguousarray(kc, np.float32)
    vc = np.ascontiguousarray(vc, np.float32)
    q = np.ascontiguousarray(q, np.float32)
    sc = np.empty(pos + 1, np.float32)
    o = np.empty(n_heads * hd, np.float32)
    lib().or_attn_decode(fptr(q), fptr(kc), fptr(vc), n_kv * hd, pos, n_heads, n_kv, hd,
                         fptr(sc), fptr(o))
    return o


def gqa_forward(Q, K, V, H, KVH, hd):
    n = Q.shape[0]
    O = np.empty((n, H * hd), np.float32)
    att = np.empty(n, np.float32)
    lib().or_gqa_forward(fptr(np.ascontiguousarray(Q, np.float32)), fptr(np.ascontiguousarray(K, np.float32)),
                         fptr(np.ascontiguousarray(V, np.float32)), n, H, KVH, hd, fptr(att), fptr(O))
    return O


def rng_create(seed):
    return int(lib().or_rng_create(seed))


def rng_uniform(state):
    """(draw, new state)"""
    st = C.c_uint64(state)
    u = lib().or_rng_uniform(C.byref(st))
    return u, st.value


def sample_token(l, temperature, top_k, top_p, state):
    """(token, new state) of sampler.c:54-143 on the float32 row l."""
    l = np.ascontiguousarray(l, np.float32)
    st = C.c_uint64(state)
    t = lib().or_sample_token(fptr(l), l.size, temperature, top_k, top_p, C.byref(st))
    return int(t), st.value


def sample_row(V, tid, sigma, kind):
    """The logits rows of the sampler fixtures: generator values, kind 1 rounded to quarters."""
    r = synth(V, 77, tid, sigma)
    if kind == 1:
        r = (np.rint(r * np.float32(4.0)) / np.float32(4.0)).astype(np.float32)
    return r


def matmul_row(a, W):
    """matrix.c:178-190 for one row: a (K,), W (K, N) f32."""
    a = np.ascontiguousarray(a, np.float32)
    W = np.ascontiguousarray(W, np.float32)
    c = np.empty(W.shape[1], np.float32)
    lib().or_matmul_row(fptr(a), fptr(W), W.shape[0], W.shape[1], fptr(c))
    return c


class FModel:
    """Oracle fp32 (LLMA) model from the generator (weights not quantized)."""

    def __init__(self, cfg, rope_base, eps=1e-5, seed=1234, tied=False):
        self.m = OrFModel()
        if lib().or_fmodel_synth(C.byref(self.m), (C.c_int32 * 8)(*cfg), rope_base, eps, seed, int(tied)) != 0:
            raise MemoryError("oracle fp32 model allocation failed")
        self.kv = OrKV()
        if lib().or_fkv_create(C.byref(self.kv), C.byref(self.m)) != 0:
            raise MemoryError("oracle kv allocation failed")
        self.vocab = cfg[0]
        self.logits = np.zeros(self.vocab, np.float32)

    def tensors(self):
        """(name, array view) in the canonical LLMA order (llama.c:198-219)."""
        m = self.m
        dm, qd, kvd, ff, V = m.d_model, m.n_heads * m.head_dim, m.n_kv * m.head_dim, m.d_ff, m.vocab
        A = lambda p, *shape: np.ctypeslib.as_array(p, shape=shape)
        out = [("wte", A(m.wte, V, dm))]
        for l in range(m.n_layers):
            b = m.blocks[l]
            out += [("attn_norm", A(b.attn_norm, dm)), ("Wq", A(b.Wq, dm, qd)), ("Wk", A(b.Wk, dm, kvd)),
                    ("Wv", A(b.Wv, dm, kvd)), ("b_q", A(b.b_q, qd)), ("b_k", A(b.b_k, kvd)),
                    ("b_v", A(b.b_v, kvd)), ("Wo", A(b.Wo, qd, dm)), ("ffn_norm", A(b.ffn_norm, dm)),
                    ("Wgate", A(b.Wgate, dm, ff)), ("Wup", A(b.Wup, dm, ff)), ("Wdown", A(b.Wdown, ff, dm))]
        return out + [("final_norm", A(m.final_norm, dm)), ("lm_head", A(m.lm_head, dm, V))]

    def hash(self):
        """The fixtures' digest: h = h*31 + hash of each tensor, canonical order."""
        h = 0
        for i, (_, t) in enumerate(self.tensors()):
            d = hash_f32(t)
            h = d if i == 0 else (h * 31 + d) & 0xFFFFFFFFFFFFFFFF
        return h

    def write_llma(self, path):
        """An 'LLMA' v2 checkpoint (llama.c:234-262): header, config, then every
        tensor's f32 values in the canonical order."""
        m = self.m
        with open(path, "wb") as f:
            f.write(struct.pack("<II", 0x414D4C4C, 2))
            f.write(struct.pack("<8i", m.vocab, m.d_model, m.n_layers, m.n_heads, m.n_kv, m.head_dim, m.d_ff,
                                m.max_seq))
            f.write(struct.pack("<2f", m.rope_base, m.eps))
            for _, t in self.tensors():
                f.write(t.astype("<f4").tobytes())

    def reset(self, length=0):
        self.kv.len = length

    def step(self, token):
        lib().or_f32_decode_step(C.byref(self.m), C.byref(self.kv), token, fptr(self.logits))
        return self.logits

    def close(self):
        if self.m.blocks:
            lib().or_kv_free(C.byref(self.kv))
            lib().or_fmodel_free(C.byref(self.m))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def layernorm(x, g, b, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().or_layernorm(fptr(x), rows, cols, fptr(np.ascontiguousarray(g, np.float32)),
                       fptr(np.ascontiguousarray(b, np.float32)), eps, fptr(y))
    return y


def gelu(x):
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    lib().or_gelu(fptr(x), x.size, fptr(y))
    return y


GPT_BLOCK = ("W_q", "W_k", "W_v", "W_o", "b_q", "b_k", "b_v", "b_o", "gamma1", "beta1", "gamma2", "beta2",
             "ff_W1", "ff_b1", "ff_W2", "ff_b2")
_GPT_FIELDS = ("Wq", "Wk", "Wv", "Wo", "bq", "bk", "bv", "bo", "g1", "be1", "g2", "be2", "W1", "bf1", "W2", "bf2")


class GPTModel:
    """Oracle GPT-2 model (model.c:437-520), weights from the generator by GPTC
    position, or zeros (synth=False) to be filled from caller arrays."""

    def __init__(self, cfg, seed=1234, synth=True):
        self.cfg = list(cfg)                     # vocab, d_model, n_heads, n_layers, d_ff, max_seq
        self.m = OrGPT()
        arr = (C.c_int32 * 6)(*cfg)
        rc = lib().or_gpt_synth(C.byref(self.m), arr, seed) if synth else lib().or_gpt_alloc(C.byref(self.m), arr)
        if rc != 0:
            raise MemoryError("oracle GPT allocation failed")
        self.kv = OrKV()
        if lib().or_gkv_create(C.byref(self.kv), C.byref(self.m)) != 0:
            raise MemoryError("oracle kv allocation failed")
        self.vocab = cfg[0]
        self.logits = np.zeros(self.vocab, np.float32)

    def tensors(self):
        """(name, array view) in the GPTC order (checkpoint.c:17-44), reference shapes."""
        m = self.m
        V, dm, ff, S = m.vocab, m.d_model, m.d_ff, m.max_seq
        A = lambda p, *shape: np.ctypeslib.as_array(p, shape=shape)
        shapes = {"W_q": (dm, dm), "W_k": (dm, dm), "W_v": (dm, dm), "W_o": (dm, dm), "ff_W1": (dm, ff),
                  "ff_b1": (ff,), "ff_W2": (ff, dm)}
        out = [("wte", A(m.wte, V, dm)), ("wpe", A(m.wpe, S, dm))]
        for l in range(m.n_layers):
            b = m.blocks[l]
            for name, fld in zip(GPT_BLOCK, _GPT_FIELDS):
                out.append((name, A(getattr(b, fld), *shapes.get(name, (dm,)))))
        return out + [("ln_f_gamma", A(m.lnf_g, dm)), ("ln_f_beta", A(m.lnf_b, dm)), ("lm_head", A(m.lm_head, dm, V))]

    def hash(self):
        return int(lib().or_gpt_hash(C.byref(self.m)))

    def write_gptc(self, path):
        """A 'GPTC' v2 checkpoint (checkpoint.c:63-112's byte order): magic, version,
        6 config ints, then every tensor's f32 values in the GPTC order."""
        m = self.m
        with open(path, "wb") as f:
            f.write(struct.pack("<II", 0x43545047, 2))
            f.write(struct.pack("<6i", m.vocab, m.d_model, m.n_heads, m.n_layers, m.d_ff, m.max_seq))
            for _, t in self.tensors():
                f.write(t.astype("<f4").tobytes())

    def reset(self, length=0):
        self.kv.len = length

    def step(self, token):
        lib().or_gpt_decode_step(C.byref(self.m), C.byref(self.kv), token, fptr(self.logits))
        return self.logits

    def close(self):
        if self.m.blocks:
            lib().or_kv_free(C.byref(self.kv))
            lib().or_gpt_free(C.byref(self.m))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def write_llmq(model, path):
    """Write an oracle Model as an 'LLMQ' v2 checkpoint: the byte order of the
    reference's reader (llama.c:603-657) and writer (tools/convert_llama.py:73-97):
    header, 8 config ints, rope base and eps, then per tensor either f32 values
    or (int8 matrices) the cols f32 scales followed by the rows*cols int8 bytes."""
    m = model.m

    def f32(ptr, n):
        return np.ctypeslib.as_array(ptr, shape=(n,)).astype("<f4").tobytes()

    def qt(t):
        return (np.ctypeslib.as_array(t.scale, shape=(t.cols,)).astype("<f4").tobytes() +
                np.ctypeslib.as_array(t.q, shape=(t.rows * t.cols,)).tobytes())

    dm, qd, kvd = m.d_model, m.n_heads * m.head_dim, m.n_kv * m.head_dim
    with open(path, "wb") as f:
        f.write(struct.pack("<II", 0x514D4C4C, 2))
        f.write(struct.pack("<8i", m.vocab, m.d_model, m.n_layers, m.n_heads, m.n_kv, m.head_dim, m.d_ff,
                            m.max_seq))
        f.write(struct.pack("<2f", m.rope_base, m.eps))
        f.write(qt(m.wte))
        for l in range(m.n_layers):
            b = m.blocks[l]
            f.write(f32(b.attn_norm, dm))
            f.write(qt(b.Wq)); f.write(qt(b.Wk)); f.write(qt(b.Wv))
            f.write(f32(b.b_q, qd)); f.write(f32(b.b_k, kvd)); f.write(f32(b.b_v, kvd))
            f.write(qt(b.Wo))
            f.write(f32(b.ffn_norm, dm))
            f.write(qt(b.Wgate)); f.write(qt(b.Wup)); f.write(qt(b.Wdown))
        f.write(f32(m.final_norm, dm))
        f.write(qt(m.lm_head))


class Model:
    """Oracle model (reference layout, host memory)."""

    def __init__(self, cfg, rope_base, eps=1e-5, seed=1234, tied=False, synth=True):
        self.m = OrModel()
        arr = (C.c_int32 * 8)(*cfg)
        if synth:
            rc = lib().or_model_synth(C.byref(self.m), arr, rope_base, eps, seed, int(tied))
        else:
            rc = lib().or_model_alloc(C.byref(self.m), arr, rope_base, eps)
        if rc != 0:
            raise MemoryError("oracle model allocation failed")
        self.kv = OrKV()
        if lib().or_kv_create(C.byref(self.kv), C.byref(self.m)) != 0:
            raise MemoryError("oracle kv allocation failed")
        self.vocab = cfg[0]
        self.logits = np.zeros(self.vocab, np.float32)

    @classmethod
    def quantize_from(cls, cfg, rope_base, eps, tensors):
        """llama.c:490-511 on an fp32 model given as (name, array) pairs in the
        canonical LLMA order (llama.c:198-219): the oracle's int8 model."""
        self = cls.__new__(cls)
        keep = []

        def P(a):
            a = np.ascontiguousarray(a, np.float32)
            keep.append(a)
            return fptr(a)

        f = OrFModel()
        (f.vocab, f.d_model, f.n_layers, f.n_heads, f.n_kv, f.head_dim, f.d_ff, f.max_seq) = cfg
        f.rope_base, f.eps = rope_base, eps
        it = iter(tensors)
        f.wte = P(next(it)[1])
        blocks = (OrFBlock * cfg[2])()
        for l in range(cfg[2]):
            for name in ("attn_norm", "Wq", "Wk", "Wv", "b_q", "b_k", "b_v", "Wo", "ffn_norm", "Wgate", "Wup", "Wdown"):
                n, a = next(it)
                assert n == name, (n, name)
                setattr(blocks[l], name, P(a))
        f.blocks = blocks
        f.final_norm = P(next(it)[1])
        f.lm_head = P(next(it)[1])
        self.m = OrModel()
        if lib().or_model_quantize_from(C.byref(self.m), C.byref(f)) != 0:
            raise MemoryError("oracle model allocation failed")
        self.kv = OrKV()
        if lib().or_kv_create(C.byref(self.kv), C.byref(self.m)) != 0:
            raise MemoryError("oracle kv allocation failed")
        self.vocab = cfg[0]
        self.logits = np.zeros(self.vocab, np.float32)
        return self

    def hash(self):
        return int(lib().or_model_hash(C.byref(self.m)))

    def reset(self, length=0):
        self.kv.len = length

    def step(self, token):
        lib().or_decode_step(C.byref(self.m), C.byref(self.kv), token, fptr(self.logits))
        return self.logits

    def close(self):
        if self.m.blocks:
            lib().or_kv_free(C.byref(self.kv))
            lib().or_model_free(C.byref(self.m))
            self.m.blocks = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
