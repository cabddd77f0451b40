"""Python host mirror of include/qllama.h (ctypes), for tests and the benchmark.

Loads the in-tree libqllama.so built by llm-project_amd/Makefile and raises if
it is missing: there is no CPU fallback.  Mirrors the reference's quantized API
(llama.h:114-140, quant.h:15-33) with numpy arrays standing in for host Tensors.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# QLLAMA_LIB selects another build of the same library (a variant for an A/B run)
LIB_PATH = os.environ.get("QLLAMA_LIB") or os.path.join(HERE, "libqllama.so")

QT_LAYOUT_NK = 0
QT_LAYOUT_KN = 1
MODE_EXACT = 0      # QLLAMA_MODE_EXACT: logits bit-identical to the reference
MODE_FAST = 1       # QLLAMA_MODE_FAST: split-K attention, tree-ordered norm sums


class Tensor(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("grad", C.POINTER(C.c_float)),
                ("shape", C.POINTER(C.c_int)), ("ndim", C.c_int), ("size", C.c_size_t)]


class QTensor(C.Structure):
    _fields_ = [("rows", C.c_int), ("cols", C.c_int), ("q", C.c_void_p), ("scale", C.c_void_p),
                ("layout", C.c_int), ("kpad", C.c_int)]


class LlamaBlock(C.Structure):
    _fields_ = [("d_model", C.c_int), ("n_heads", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("d_ff", C.c_int), ("rope_base", C.c_float), ("eps", C.c_float)] + \
               [(n, Tensor) for n in ("attn_norm", "Wq", "Wk", "Wv", "b_q", "b_k", "b_v", "Wo",
                                      "ffn_norm", "Wgate", "Wup", "Wdown")]


class LlamaModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "d_model", "n_layers", "n_heads", "n_kv", "head_dim",
                                       "d_ff", "max_seq")] + \
               [("rope_base", C.c_float), ("eps", C.c_float), ("wte", Tensor),
                ("blocks", C.POINTER(LlamaBlock)), ("final_norm", Tensor), ("lm_head", Tensor)]


class LlamaKV(C.Structure):
    _fields_ = [("n_layers", C.c_int), ("max_seq", C.c_int), ("kv_dim", C.c_int), ("len", C.c_int),
                ("k", C.POINTER(C.c_void_p)), ("v", C.POINTER(C.c_void_p)), ("dev", C.c_void_p)]


class QLlamaBlock(C.Structure):
    _fields_ = [("attn_norm", Tensor), ("ffn_norm", Tensor), ("b_q", Tensor), ("b_k", Tensor),
                ("b_v", Tensor)] + [(n, QTensor) for n in ("Wq", "Wk", "Wv", "Wo", "Wgate", "Wup", "Wdown")]


class BlockWeights(C.Structure):               # model.h:8-16
    _fields_ = [(n, Tensor) for n in ("W_q", "W_k", "W_v", "W_o", "b_q", "b_k", "b_v", "b_o", "gamma1", "beta1",
                                      "gamma2", "beta2", "ff_W1", "ff_b1", "ff_W2", "ff_b2")]


class GPT(C.Structure):                        # model.h:19-31
    _fields_ = [(n, C.c_int) for n in ("vocab_size", "d_model", "n_heads", "n_layers", "d_ff", "max_seq_len")] + \
               [("wte", Tensor), ("wpe", Tensor), ("blocks", C.POINTER(BlockWeights)), ("ln_f_gamma", Tensor),
                ("ln_f_beta", Tensor), ("lm_head", Tensor)]


class KVCache(C.Structure):                    # model.h:124-129 + the device handle
    _fields_ = [(n, C.c_int) for n in ("n_layers", "d_model", "n_heads", "max_seq_len", "len")] + \
               [("K", C.POINTER(Tensor)), ("V", C.POINTER(Tensor)), ("dev", C.c_void_p)]


class Rng(C.Structure):
    _fields_ = [("state", C.c_ulonglong)]        # sampler.h:15-17


class QLlamaModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("vocab", "d_model", "n_layers", "n_heads", "n_kv", "head_dim",
                                       "d_ff", "max_seq")] + \
               [("rope_base", C.c_float), ("eps", C.c_float), ("wte", QTensor),
                ("blocks", C.POINTER(QLlamaBlock)), ("final_norm", Tensor), ("lm_head", QTensor),
                ("dev", C.c_void_p)]


_lib = None


def lib():
    """The loaded libqllama.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C llm-project_amd` "
                               "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        P = C.POINTER
        L.q_llama_model_load.argtypes = [C.c_char_p, P(QLlamaModel)]
        L.q_llama_model_free.argtypes = [P(QLlamaModel)]
        L.q_llama_quantize_from.argtypes = [P(LlamaModel)]
        L.q_llama_quantize_from.restype = QLlamaModel
        L.q_llama_kv_create.argtypes = [P(QLlamaModel)]
        L.q_llama_kv_create.restype = LlamaKV
        L.q_llama_kv_create_mode.argtypes = [P(QLlamaModel), C.c_int]
        L.q_llama_kv_create_mode.restype = LlamaKV
        L.llama_kv_free.argtypes = [P(LlamaKV)]
        L.q_llama_decode_step.argtypes = [P(QLlamaModel), P(LlamaKV), C.c_int, P(Tensor)]
        L.q_llama_prefill.argtypes = [P(QLlamaModel), P(LlamaKV), P(C.c_int), C.c_int, P(Tensor)]
        L.q_llama_generate_greedy.argtypes = [P(QLlamaModel), P(LlamaKV), C.c_int, C.c_int, P(C.c_int)]
        L.q_llama_model_synth.argtypes = [P(QLlamaModel), P(C.c_int32), C.c_float, C.c_float, C.c_uint64, C.c_int]
        L.q_llama_model_hash.argtypes = [P(QLlamaModel)]
        L.q_llama_model_hash.restype = C.c_uint64
        L.qtensor_create.argtypes = [C.c_int, C.c_int]
        L.qtensor_create.restype = QTensor
        L.qtensor_free.argtypes = [P(QTensor)]
        L.qtensor_quantize.argtypes = [P(QTensor), P(C.c_float)]
        L.qmatmul.argtypes = [P(Tensor), P(QTensor), P(Tensor)]
        L.quantize_int8_percol.argtypes = [P(C.c_float), C.c_int, C.c_int, P(C.c_int8), P(C.c_float)]
        L.dequantize_int8_percol.argtypes = [P(C.c_int8), P(C.c_float), C.c_int, C.c_int, P(C.c_float)]
        L.qacc_columns.argtypes = [P(C.c_int8), P(C.c_int8), C.c_int, C.c_int, P(C.c_int32)]
        L.q_llama_model_save.argtypes = [P(QLlamaModel), C.c_char_p]
        L.q_llama_tensor_export.argtypes = [P(QTensor), P(C.c_int8), P(C.c_float)]
        L.llama_kv_create.argtypes = [P(LlamaModel)]
        L.llama_kv_create.restype = LlamaKV
        L.llama_decode_step.argtypes = [P(LlamaModel), P(LlamaKV), C.c_int, P(Tensor)]
        L.llama_model_forward.argtypes = [P(LlamaModel), P(C.c_int), C.c_int, P(Tensor)]
        L.rng_create.argtypes = [C.c_ulonglong]
        L.rng_create.restype = Rng
        L.rng_uniform.argtypes = [P(Rng)]
        L.rng_uniform.restype = C.c_float
        L.sample_argmax.argtypes = [P(Tensor), C.c_int]
        L.sample_token.argtypes = [P(Tensor), C.c_int, C.c_float, C.c_int, C.c_float, P(Rng)]
        L.q_llama_generate.argtypes = [P(QLlamaModel), P(LlamaKV), C.c_int, C.c_float, C.c_int, C.c_float, P(Rng),
                                       P(C.c_int)]
        L.gpt_load.argtypes = [C.c_char_p, P(GPT)]
        L.gpt_save.argtypes = [C.c_char_p, P(GPT)]
        L.gpt_free.argtypes = [P(GPT)]
        L.gpt_kvcache_refresh.argtypes = [P(KVCache), P(GPT)]
        L.gpt_kvcache_refresh.restype = C.c_int
        L.gpt_kvcache_create.argtypes = [P(GPT)]
        L.gpt_kvcache_create.restype = KVCache
        L.gpt_kvcache_free.argtypes = [P(KVCache)]
        L.gpt_decode_step.argtypes = [P(GPT), P(KVCache), C.c_int, P(Tensor)]
        L.qllama_test_tanhf.argtypes = [C.c_uint32, C.c_uint32, P(C.c_float)]
        L.qtensor_synth.argtypes = [C.c_int, C.c_int, C.c_uint64, C.c_uint64, C.c_double]
        L.qtensor_synth.restype = QTensor
        L.qllama_bench_qmatmul.argtypes = [P(QTensor), C.c_int, C.c_int] + [P(C.c_double)] * 3
        L.qllama_device_count.restype = C.c_int
        L.qllama_dev_alloc.argtypes = [C.c_size_t]
        L.qllama_dev_alloc.restype = C.c_void_p
        L.qllama_dev_free.argtypes = [C.c_void_p]
        L.qllama_h2d.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        L.qllama_d2h.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        L.qllama_device_sync.restype = C.c_int
        L.qllama_test_expf.argtypes = [C.c_uint32, C.c_uint32, P(C.c_float)]
        L.qllama_gqa_decode.argtypes = [P(C.c_float)] * 3 + [C.c_int] * 4 + [P(C.c_float)]
        L.qllama_norm_gemv.argtypes = [P(C.c_float), P(C.c_float), C.c_float, P(QTensor), C.c_int, C.c_int,
                                       P(C.c_float)]
        L.qllama_gqa_decode_ex.argtypes = [P(C.c_float)] * 3 + [C.c_int] * 4 + [C.c_float, C.c_int, C.c_int] + \
            [P(C.c_float), P(C.c_float), P(C.c_double)]
        L.qllama_pf_attention_ex.argtypes = [P(C.c_float)] * 3 + [C.c_int] * 7 + [P(C.c_float), P(C.c_double)]
        L.qllama_sync.restype = C.c_int
        L.qllama_attn_layer_active.argtypes = [P(QLlamaModel)]
        L.qllama_attn_layer_active.restype = C.c_int
        L.qllama_stream.restype = C.c_void_p
        L.qllama_profile.argtypes = [C.c_int]
        L.qllama_bench_cold.argtypes = [C.c_int]
        L.qllama_profile_read.argtypes = [C.c_char_p, C.c_int, P(C.c_double), P(C.c_longlong), C.c_int]
        _lib = L
    return _lib


def _f32(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def host_tensor(a):
    """A reference Tensor view of a C-contiguous float32 numpy array (kept alive by the caller)."""
    assert a.dtype == np.float32 and a.flags.c_contiguous
    shape = (C.c_int * a.ndim)(*a.shape)
    t = Tensor(_f32(a), None, shape, a.ndim, a.size)
    t._keep = (a, shape)
    return t


class Model:
    """A QLlamaModel plus one LlamaKV (decode mode chosen at creation), on the GPU.
    fork(mode) gives another cache on the same device weights."""

    def __init__(self, m, mode=MODE_EXACT, owner=None):
        self.m = m
        self.mode = mode
        self._owner = owner          # the Model that owns the weights, for forks
        self.kv = lib().q_llama_kv_create_mode(C.byref(self.m), mode)
        self.vocab = m.vocab
        self.logits = np.zeros((1, m.vocab), np.float32)
        self._lt = host_tensor(self.logits)

    @classmethod
    def synth(cls, cfg, rope_base, eps=1e-5, seed=1234, tied=False, mode=MODE_EXACT):
        m = QLlamaModel()
        arr = (C.c_int32 * 8)(*cfg)
        if lib().q_llama_model_synth(C.byref(m), arr, rope_base, eps, seed, int(tied)) != 0:
            raise RuntimeError("q_llama_model_synth failed")
        return cls(m, mode)

    @classmethod
    def load(cls, path, mode=MODE_EXACT):
        m = QLlamaModel()
        if lib().q_llama_model_load(os.fsencode(path), C.byref(m)) != 0:
            raise RuntimeError(f"q_llama_model_load failed for {path}")
        return cls(m, mode)

    @classmethod
    def quantize_from(cls, cfg, rope_base, eps, tensors, mode=MODE_EXACT):
        """q_llama_quantize_from (llama.c:490-511) of a host fp32 LlamaModel given
        as (name, array) pairs in the canonical LLMA order (llama.c:198-219)."""
        host = host_model(cfg, rope_base, eps, tensors)
        m = lib().q_llama_quantize_from(C.byref(host))
        return cls(m, mode)

    def fork(self, mode):
        """A second cache (q_llama_kv_create_mode) on this model's device weights;
        close it before the model."""
        return Model(self.m, mode, owner=self)

    @property
    def pos(self):
        return self.kv.len

    def reset(self, length=0):
        self.kv.len = length

    def hash(self):
        return int(lib().q_llama_model_hash(C.byref(self.m)))

    def attn_layer_active(self):
        """Whether the exact decode steps run each layer's attention half
        (QKV, RoPE, cache append, scores, softmax, PV) as one launch."""
        return bool(lib().qllama_attn_layer_active(C.byref(self.m)))

    def step(self, token):
        lib().q_llama_decode_step(C.byref(self.m), C.byref(self.kv), int(token), C.byref(self._lt))
        return self.logits[0]

    def prefill(self, ids, want_logits=True):
        arr = (C.c_int * len(ids))(*ids)
        rc = lib().q_llama_prefill(C.byref(self.m), C.byref(self.kv), arr, len(ids),
                                   C.byref(self._lt) if want_logits else None)
        if rc != 0:
            raise RuntimeError("q_llama_prefill failed")
        return self.logits[0]

    def generate_greedy(self, token, n):
        out = (C.c_int * n)()
        if lib().q_llama_generate_greedy(C.byref(self.m), C.byref(self.kv), int(token), n, out) != 0:
            raise RuntimeError("q_llama_generate_greedy failed")
        return list(out)

    def save(self, path):
        """Write an LLMQ v2 checkpoint (q_llama_model_save)."""
        if lib().q_llama_model_save(C.byref(self.m), os.fsencode(path)) != 0:
            raise RuntimeError(f"q_llama_model_save failed for {path}")

    def generate(self, n, temperature, top_k, top_p, rng):
        """n sampled tokens (q_llama_generate); rng is an Rng, advanced in place."""
        out = (C.c_int * n)()
        if lib().q_llama_generate(C.byref(self.m), C.byref(self.kv), n, temperature, top_k, top_p,
                                  C.byref(rng), out) != 0:
            raise RuntimeError("q_llama_generate failed")
        return list(out)

    def close(self):
        if self._owner is not None:
            if self.kv.dev:
                lib().llama_kv_free(C.byref(self.kv))
                self.kv.dev = None
            return
        if self.m.dev:
            lib().llama_kv_free(C.byref(self.kv))
            lib().q_llama_model_free(C.byref(self.m))
            self.m.dev = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- fp32 (LLMA) path -----------------------------------------------------------
def host_model(cfg, rope_base, eps, tensors):
    """A reference LlamaModel (host memory) over float32 arrays given in the
    canonical order of llama.c:198-219 as (name, array) pairs; the arrays are
    kept alive by the returned object."""
    keep = []

    def T(a):
        a = np.ascontiguousarray(a, np.float32)
        keep.append(a)
        t = host_tensor(a)
        keep.append(t._keep)
        return t

    m = LlamaModel()
    (m.vocab, m.d_model, m.n_layers, m.n_heads, m.n_kv, m.head_dim, m.d_ff, m.max_seq) = cfg
    m.rope_base, m.eps = rope_base, eps
    it = iter(tensors)
    m.wte = T(next(it)[1])
    blocks = (LlamaBlock * cfg[2])()
    for l in range(cfg[2]):
        b = blocks[l]
        b.d_model, b.n_heads, b.n_kv, b.head_dim, b.d_ff = cfg[1], cfg[3], cfg[4], cfg[5], cfg[6]
        b.rope_base, b.eps = rope_base, eps
        for name in ("attn_norm", "Wq", "Wk", "Wv", "b_q", "b_k", "b_v", "Wo", "ffn_norm", "Wgate", "Wup", "Wdown"):
            n, a = next(it)
            assert n == name, (n, name)
            setattr(b, name, T(a))
    m.blocks = blocks
    m.final_norm = T(next(it)[1])
    m.lm_head = T(next(it)[1])
    m._keep = (keep, blocks)
    return m


class FModel:
    """fp32 decode on the GPU (llama_kv_create / llama_decode_step) of a host LlamaModel."""

    def __init__(self, host):
        self.m = host
        self.kv = lib().llama_kv_create(C.byref(self.m))
        self.logits = np.zeros((1, host.vocab), np.float32)
        self._lt = host_tensor(self.logits)

    @property
    def pos(self):
        return self.kv.len

    def reset(self, length=0):
        self.kv.len = length

    def step(self, token):
        lib().llama_decode_step(C.byref(self.m), C.byref(self.kv), int(token), C.byref(self._lt))
        return self.logits[0]

    def forward(self, ids):
        """llama_model_forward: (len(ids), vocab) logits of every position."""
        out = np.zeros((len(ids), self.m.vocab), np.float32)
        arr = (C.c_int * len(ids))(*ids)
        lib().llama_model_forward(C.byref(self.m), arr, len(ids), C.byref(host_tensor(out)))
        return out

    def close(self):
        if self.kv.dev:
            lib().llama_kv_free(C.byref(self.kv))
            self.kv.dev = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---- GPT-2 (GPTC) path ------------------------------------------------------------
GPT_BLOCK = ("W_q", "W_k", "W_v", "W_o", "b_q", "b_k", "b_v", "b_o", "gamma1", "beta1", "gamma2", "beta2",
             "ff_W1", "ff_b1", "ff_W2", "ff_b2")


def host_gpt(cfg, tensors):
    """A reference GPT (host memory, model.h:19-31) over float32 arrays given in
    the GPTC order (checkpoint.c:17-44) as (name, array) pairs; cfg = (vocab,
    d_model, n_heads, n_layers, d_ff, max_seq).  The arrays are kept alive by
    the returned object."""
    keep = []

    def T(a):
        a = np.ascontiguousarray(a, np.float32)
        keep.append(a)
        t = host_tensor(a)
        keep.append(t._keep)
        return t

    m = GPT()
    (m.vocab_size, m.d_model, m.n_heads, m.n_layers, m.d_ff, m.max_seq_len) = cfg
    it = iter(tensors)
    m.wte = T(next(it)[1])
    m.wpe = T(next(it)[1])
    blocks = (BlockWeights * cfg[3])()
    for l in range(cfg[3]):
        for name in GPT_BLOCK:
            n, a = next(it)
            assert n == name, (n, name)
            setattr(blocks[l], name, T(a))
    m.blocks = blocks
    m.ln_f_gamma = T(next(it)[1])
    m.ln_f_beta = T(next(it)[1])
    m.lm_head = T(next(it)[1])
    m._keep = (keep, blocks)
    return m


class GPTDecoder:
    """gpt_kvcache_create / gpt_decode_step of a host GPT, on the GPU."""

    def __init__(self, host):
        self.m = host
        self.kv = lib().gpt_kvcache_create(C.byref(self.m))
        self.logits = np.zeros((1, host.vocab_size), np.float32)
        self._lt = host_tensor(self.logits)

    @property
    def pos(self):
        return self.kv.len

    def reset(self, length=0):
        self.kv.len = length

    def step(self, token):
        lib().gpt_decode_step(C.byref(self.m), C.byref(self.kv), int(token), C.byref(self._lt))
        return self.logits[0]

    def close(self):
        if self.kv.dev:
            lib().gpt_kvcache_free(C.byref(self.kv))
            self.kv.dev = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def ctypes_byref(obj):
    return C.byref(obj)


def gpt_load(path):
    """checkpoint.c gpt_load into a host GPT (free it with gpt_free)."""
    m = GPT()
    if lib().gpt_load(os.fsencode(path), C.byref(m)) != 0:
        raise RuntimeError(f"gpt_load failed for {path}")
    return m


def gpt_tensors(m):
    """(name, array view) of a host GPT in the GPTC order."""
    V, dm, ff, S = m.vocab_size, m.d_model, m.d_ff, m.max_seq_len
    A = lambda t, *shape: np.ctypeslib.as_array(t.data, shape=shape)
    shapes = {"W_q": (dm, dm), "W_k": (dm, dm), "W_v": (dm, dm), "W_o": (dm, dm), "ff_W1": (dm, ff),
              "ff_b1": (ff,), "ff_W2": (ff, dm)}
    out = [("wte", A(m.wte, V, dm)), ("wpe", A(m.wpe, S, dm))]
    for l in range(m.n_layers):
        for name in GPT_BLOCK:
            out.append((name, A(getattr(m.blocks[l], name), *shapes.get(name, (dm,)))))
    return out + [("ln_f_gamma", A(m.ln_f_gamma, dm)), ("ln_f_beta", A(m.ln_f_beta, dm)),
                  ("lm_head", A(m.lm_head, dm, V))]


# ---- sampler.h API ----------------------------------------------------------
def rng_create(seed):
    return lib().rng_create(seed)


def sample_token(logits, temperature, top_k, top_p, rng, row=0):
    """sample_token on a (rows, vocab) float32 array (sampled on the GPU); rng advances in place."""
    a = np.ascontiguousarray(logits, np.float32).reshape(-1, logits.shape[-1])
    return int(lib().sample_token(C.byref(host_tensor(a)), row, temperature, top_k, top_p, C.byref(rng)))


def sample_argmax(logits, row=0):
    a = np.ascontiguousarray(logits, np.float32).reshape(-1, logits.shape[-1])
    return int(lib().sample_argmax(C.byref(host_tensor(a)), row))


# ---- quant.h API ------------------------------------------------------------
class QWeight:
    """A device QTensor (quant.h:22-27) quantized from a host (rows, cols) f32 matrix."""

    def __init__(self, w):
        w = np.ascontiguousarray(w, np.float32)
        self.rows, self.cols = w.shape
        self.t = lib().qtensor_create(self.rows, self.cols)
        lib().qtensor_quantize(C.byref(self.t), _f32(w))

    def close(self):
        if self.t.q:
            lib().qtensor_free(C.byref(self.t))
            self.t.q = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def qmatmul(A, W):
    A = np.ascontiguousarray(A, np.float32)
    Cm = np.zeros((A.shape[0], W.cols), np.float32)
    ta, tc = host_tensor(A), host_tensor(Cm)
    lib().qmatmul(C.byref(ta), C.byref(W.t), C.byref(tc))
    return Cm


def quantize_int8_percol(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    q = np.zeros((rows, cols), np.int8)
    s = np.zeros(cols, np.float32)
    lib().quantize_int8_percol(_f32(w), rows, cols, q.ctypes.data_as(C.POINTER(C.c_int8)), _f32(s))
    return q, s


def dequantize_int8_percol(q, s):
    q = np.ascontiguousarray(q, np.int8)
    s = np.ascontiguousarray(s, np.float32)
    rows, cols = q.shape
    w = np.zeros((rows, cols), np.float32)
    lib().dequantize_int8_percol(q.ctypes.data_as(C.POINTER(C.c_int8)), _f32(s), rows, cols, _f32(w))
    return w


def qacc_columns(qa, qw):
    qa = np.ascontiguousarray(qa, np.int8)
    qw = np.ascontiguousarray(qw, np.int8)
    K, N = qw.shape
    acc = np.zeros(N, np.int32)
    lib().qacc_columns(qa.ctypes.data_as(C.POINTER(C.c_int8)), qw.ctypes.data_as(C.POINTER(C.c_int8)), K, N,
                       acc.ctypes.data_as(C.POINTER(C.c_int32)))
    return acc


def norm_gemv(x, gamma, W, mode=0, fast=False, eps=1e-5):
    """qllama_norm_gemv: rmsnorm + quantization of the row x inside the decode
    GEMV against the QWeight W (mode 0 plain, 2 SwiGLU over W's column halves)."""
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    out = np.zeros(W.cols // 2 if mode == 2 else W.cols, np.float32)
    if lib().qllama_norm_gemv(_f32(x), _f32(g), eps, C.byref(W.t), mode, int(bool(fast)), _f32(out)) != 0:
        raise RuntimeError("qllama_norm_gemv failed")
    return out


def gqa_decode(q, k, v, n_heads, n_kv, hd, mode=MODE_EXACT, rope_base=0.0, reps=0):
    """qllama_gqa_decode_ex: decode attention of position T-1 over T cached rows
    (k, v: (T, n_kv*hd) in the reference's layout).  With rope_base > 0, q and
    rows T-1 of k and v are unrotated and the device applies RoPE and the cache
    append.  Returns (o, rotated k row T-1 as cached, microseconds per call or None)."""
    q = np.ascontiguousarray(q, np.float32).ravel()
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    T = k.shape[0]
    o = np.zeros(n_heads * hd, np.float32)
    krow = np.zeros(n_kv * hd, np.float32)
    us = C.c_double(0.0)
    rc = lib().qllama_gqa_decode_ex(_f32(q), _f32(k), _f32(v), T, n_heads, n_kv, hd, float(rope_base), int(mode),
                                    int(reps), _f32(o), _f32(krow), C.byref(us))
    if rc != 0:
        raise RuntimeError("qllama_gqa_decode_ex failed")
    return o, krow, (us.value if reps else None)


def pf_attention(q, k, v, n_heads, n_kv, hd, p0=0, mode=MODE_EXACT, reps=0):
    """qllama_pf_attention_ex: causal attention of the R rows of q (rotated, at
    positions p0 .. p0+R-1) over the p0+R rows of k, v (reference layout).
    Returns (o of shape (R, n_heads*hd), microseconds per call or None)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    R = q.shape[0]
    assert k.shape[0] == p0 + R and v.shape == k.shape
    o = np.zeros((R, n_heads * hd), np.float32)
    us = C.c_double(0.0)
    rc = lib().qllama_pf_attention_ex(_f32(q), _f32(k), _f32(v), R, p0, n_heads, n_kv, hd, int(mode), int(reps),
                                      _f32(o), C.byref(us))
    if rc != 0:
        raise RuntimeError("qllama_pf_attention_ex failed")
    return o, (us.value if reps else None)


PROFILE_SERIAL, PROFILE_COLD = 3, 5


def profile(enable):
    """enable: False/0 off, True/1 on, PROFILE_SERIAL (each timed launch on a
    drained stream), PROFILE_COLD (serialized, behind a 512 MB read each)."""
    lib().qllama_profile(int(enable))


def bench_cold(on):
    """Cold op-level timing of qllama_bench_qmatmul / gqa_decode(reps=...)."""
    lib().qllama_bench_cold(1 if on else 0)


def profile_read():
    names = C.create_string_buffer(4096)
    ms = (C.c_double * 32)()
    cnt = (C.c_longlong * 32)()
    n = lib().qllama_profile_read(names, 4096, ms, cnt, 32)
    keys = names.value.decode().split(",")[:max(n, 0)]
    return {k: (ms[i], cnt[i]) for i, k in enumerate(keys)}
