"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py to check and time against. See oracle.h for the reference
file:line each function restates and for what pins it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


class OrTensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("ndim", C.c_uint32),
                ("shape", C.c_uint64 * 4), ("data", C.c_void_p), ("nbytes", C.c_uint64)]


class OrMeta(C.Structure):
    _fields_ = [("n_head", C.c_uint32), ("n_layer", C.c_uint32), ("n_ctx", C.c_uint32),
                ("n_state", C.c_uint32), ("n_vocab", C.c_uint32)]


class OrEncMeta(C.Structure):
    _fields_ = [("n_head", C.c_uint32), ("n_layer", C.c_uint32), ("n_ctx", C.c_uint32),
                ("n_state", C.c_uint32), ("n_mels", C.c_uint32)]


class OrDecodeParams(C.Structure):
    _fields_ = [("prompt", C.POINTER(C.c_int32)), ("prompt_len", C.c_int32), ("beam_size", C.c_int32),
                ("temperature", C.c_float), ("logprob_thold", C.c_float), ("no_speech_thold", C.c_float),
                ("no_fallback", C.c_int32), ("max_tokens", C.c_int32), ("suppress_nst", C.c_int32)]


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        L = C.CDLL(_SO)
        P = C.c_void_p
        sig = {
            "or_f16_to_f32": (C.c_float, [C.c_uint16]),
            "or_f32_to_f16": (C.c_uint16, [C.c_float]),
            "or_row_bytes": (C.c_size_t, [C.c_uint32, C.c_size_t]),
            "or_dequantize": (C.c_int, [P, C.c_uint32, C.c_size_t, P]),
            "or_quantize": (C.c_size_t, [P, C.c_size_t, C.c_uint32, P]),
            "or_should_quantize": (C.c_int, [C.c_char_p]),
            "or_dot": (C.c_float, [C.c_uint32, P, P, C.c_int, C.c_int]),
            "or_gemv": (C.c_int, [C.c_uint32, P, C.c_int, C.c_int, P, C.c_int, P, C.c_int, C.c_int]),
            "or_layernorm": (None, [P, P, P, P, C.c_int, C.c_int, C.c_float]),
            "or_gelu": (None, [P, C.c_int]),
            "or_fast_exp": (C.c_float, [C.c_float]),
            "or_softmax_fast": (None, [P, C.c_int]),
            "or_softmax_exact": (None, [P, C.c_int]),
            "or_sdpa": (None, [P, P, P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, P, P]),
            "or_repetition_penalty": (None, [P, C.c_int, P, C.c_int, C.c_float, C.c_int, P]),
            "or_sample_greedy": (C.c_int32, [P, C.c_int, C.c_float, C.c_int, C.c_float, C.c_int32]),
            "or_topk": (C.c_int, [P, C.c_int, C.c_int, C.c_float, P, P]),
            "or_model_create": (P, [C.POINTER(OrTensor), C.c_int, C.POINTER(OrMeta), C.c_int, C.c_int]),
            "or_model_destroy": (None, [P]),
            "or_model_hparams": (None, [P, P]),
            "or_model_set_eot": (None, [P, C.c_int32]),
            "or_model_set_fast_exp": (None, [P, C.c_int]),
            "or_model_set_forward_threads": (None, [P, C.c_int]),
            "or_state_create": (P, [P, P, C.c_int]),
            "or_state_destroy": (None, [P]),
            "or_state_reset": (None, [P, P, P, C.c_int]),
            "or_state_push": (C.c_int, [P, C.c_int32]),
            "or_forward": (C.c_int, [P, P, P, C.c_int, P]),
            "or_state_prepare_cross": (C.c_int, [P, P, P, C.c_int]),
            "or_decode": (C.c_int, [P, P, C.c_int, C.POINTER(OrDecodeParams), P, C.c_int, P]),
            "or_beam_run": (C.c_int, [P, P, C.c_int, C.POINTER(OrDecodeParams), P, C.c_int, P, P, P, P, C.c_int]),
            "or_go_sort_norm": (None, [P, P, C.c_int]),
            "or_encoder_create": (P, [C.POINTER(OrTensor), C.c_int, C.POINTER(OrEncMeta), C.c_int, C.c_int]),
            "or_encoder_destroy": (None, [P]),
            "or_encoder_hparams": (None, [P, P]),
            "or_encoder_set_fast_exp": (None, [P, C.c_int]),
            "or_encode": (C.c_int, [P, P, C.c_int, C.c_int, P]),
            "or_conv1d": (C.c_int, [P, C.c_int, C.c_int, P, P, C.c_int, C.c_int, C.c_int, P]),
            "or_last_error": (C.c_char_p, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data


def f16_to_f32(h):
    return lib().or_f16_to_f32(int(h))


def f32_to_f16(f):
    return lib().or_f32_to_f16(float(f))


def row_bytes(qtype, n):
    return lib().or_row_bytes(qtype, n)


def dequantize(raw, qtype, n):
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty(n, np.float32)
    if lib().or_dequantize(_p(raw), qtype, n, _p(out)) != 0:
        raise RuntimeError(lib().or_last_error().decode())
    return out


def quantize(x, qtype):
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(row_bytes(qtype, x.size), np.uint8)
    lib().or_quantize(_p(x), x.size, qtype, _p(out))
    return out


def should_quantize(name):
    return bool(lib().or_should_quantize(name.encode()))


def dot(qtype, row, x, variant=1):
    row = np.ascontiguousarray(row, np.uint8) if qtype != 0 else np.ascontiguousarray(row, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    return lib().or_dot(qtype, _p(row), _p(x), x.size, variant)


def gemv(qtype, w, rows, cols, a, variant=1, threads=1):
    a = np.ascontiguousarray(a, np.float32).reshape(-1, cols)
    w = np.ascontiguousarray(w)
    out = np.empty((a.shape[0], rows), np.float32)
    if lib().or_gemv(qtype, _p(w), rows, cols, _p(a), a.shape[0], _p(out), variant, threads) != 0:
        raise RuntimeError(lib().or_last_error().decode())
    return out


def layernorm(x, w, b, eps=1e-5):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty_like(x)
    c = x.shape[-1]
    lib().or_layernorm(_p(out), _p(x), _p(w), _p(b), x.size // c, c, eps)
    return out


def gelu(x):
    x = np.array(x, np.float32, copy=True).reshape(-1)
    lib().or_gelu(_p(x), x.size)
    return x


def fast_exp(x):
    return lib().or_fast_exp(float(x))


def softmax(row, fast=True):
    r = np.array(row, np.float32, copy=True)
    (lib().or_softmax_fast if fast else lib().or_softmax_exact)(_p(r), r.size)
    return r


def sdpa(q, k, v, causal, fast=True, weights=False):
    q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
    H, tq, hd = q.shape
    tk = k.shape[1]
    out = np.empty_like(q)
    w = np.empty((H, tq, tk), np.float32) if weights else None
    lib().or_sdpa(_p(q), _p(k), _p(v), H, tq, tk, hd, int(causal), int(fast), _p(out), _p(w) if weights else None)
    return (out, w) if weights else out


def repetition_penalty(logits, hist, penalty=2.0, window=128):
    l = np.ascontiguousarray(logits, np.float32)
    h = np.ascontiguousarray(hist, np.int32)
    out = np.empty_like(l)
    lib().or_repetition_penalty(_p(l), l.size, _p(h), h.size, penalty, window, _p(out))
    return out


def sample_greedy(logits, temperature=1.0, suppress_nst=False, no_speech_thold=0.0, eot=50256):
    l = np.ascontiguousarray(logits, np.float32)
    return lib().or_sample_greedy(_p(l), l.size, temperature, int(suppress_nst), no_speech_thold, eot)


def topk(logits, k, temperature=1.0):
    l = np.ascontiguousarray(logits, np.float32)
    tok = np.empty(k, np.int32)
    lp = np.empty(k, np.float32)
    n = lib().or_topk(_p(l), l.size, k, temperature, _p(tok), _p(lp))
    return tok[:n], lp[:n]


def go_sort_norm(norm, ids=None):
    """Go's sort.Slice by norm descending (pdqsort); returns (norm, ids) in the sorted order."""
    n = np.array(norm, np.float32, copy=True)
    i = np.arange(n.size, dtype=np.int32) if ids is None else np.array(ids, np.int32, copy=True)
    lib().or_go_sort_norm(_p(n), _p(i), n.size)
    return n, i


def _params(params):
    prompt = (C.c_int32 * max(1, len(params.prompt)))(*params.prompt)
    p = OrDecodeParams(C.cast(prompt, C.POINTER(C.c_int32)), len(params.prompt), params.beam_size,
                       params.temperature, params.logprob_thold, params.no_speech_thold,
                       int(params.no_fallback), params.max_tokens, int(params.suppress_nst))
    return p, prompt


class OracleModel:
    """or_model over a tensor table (objects with .name .type .shape .data)."""

    def __init__(self, tensors, meta=None, dot_variant=1, threads=1):
        self._keep = []
        arr = (OrTensor * len(tensors))()
        for i, t in enumerate(tensors):
            name = t.name.encode()
            data = np.ascontiguousarray(t.data)
            self._keep += [name, data]
            arr[i].name, arr[i].type, arr[i].ndim = name, t.type, len(t.shape)
            for j, s in enumerate(t.shape):
                arr[i].shape[j] = s
            arr[i].data, arr[i].nbytes = data.ctypes.data, data.size
        self._arr = arr
        m = OrMeta(**(meta or {}))
        self._h = lib().or_model_create(arr, len(tensors), C.byref(m), dot_variant, threads)
        if not self._h:
            raise RuntimeError(lib().or_last_error().decode())
        hp = np.zeros(5, np.int32)
        lib().or_model_hparams(self._h, _p(hp))
        self.n_vocab, self.n_state, self.n_head, self.n_layer, self.n_ctx = (int(v) for v in hp)
        self.eot = 50256

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_model_destroy(self._h)
            self._h = None

    def set_eot(self, eot):
        lib().or_model_set_eot(self._h, eot)
        self.eot = eot

    def set_fast_exp(self, on):
        lib().or_model_set_fast_exp(self._h, int(on))

    def set_forward_threads(self, n):
        lib().or_model_set_forward_threads(self._h, int(n))

    def state(self, tokens):
        return OracleState(self, tokens)

    def decode(self, enc, params):
        enc = np.ascontiguousarray(enc, np.float32)
        p, _keep = _params(params)
        cap = len(params.prompt) + max(1, params.beam_size) * (self.n_ctx + 1) + 8
        out = np.empty(cap, np.int32)
        n = C.c_int32()
        if lib().or_decode(self._h, _p(enc), enc.shape[0], C.byref(p), _p(out), cap, C.byref(n)) != 0:
            raise RuntimeError(lib().or_last_error().decode())
        return [int(t) for t in out[:n.value]]

    def beam_run(self, enc, params, margins=False):
        """Every beam after the search: [(tokens, score)] in the final beams order
        (and, with margins=True, the per-step selection margins)."""
        enc = np.ascontiguousarray(enc, np.float32)
        p, _keep = _params(params)
        bs = max(1, params.beam_size)
        cap = len(params.prompt) + bs * (self.n_ctx + 1) + 8
        out = np.zeros((bs, cap), np.int32)
        lens = np.zeros(bs, np.int32)
        scores = np.zeros(bs, np.float32)
        marg = np.full(self.n_ctx + 1, np.nan, np.float32)
        nb = C.c_int32()
        if lib().or_beam_run(self._h, _p(enc), enc.shape[0], C.byref(p), _p(out), cap, _p(lens), _p(scores),
                             C.byref(nb), _p(marg), marg.size) != 0:
            raise RuntimeError(lib().or_last_error().decode())
        beams = [([int(t) for t in out[i, :lens[i]]], float(scores[i])) for i in range(nb.value)]
        if margins:
            return beams, [float(m) for m in marg if not np.isnan(m)]
        return beams


class OracleState:
    def __init__(self, model, tokens):
        self.m = model
        t = np.ascontiguousarray(tokens, np.int32)
        self._h = lib().or_state_create(model._h, _p(t), t.size)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_state_destroy(self._h)
            self._h = None

    def push(self, tok):
        lib().or_state_push(self._h, int(tok))

    def reset(self, tokens):
        t = np.ascontiguousarray(tokens, np.int32)
        lib().or_state_reset(self.m._h, self._h, _p(t), t.size)

    def prepare_cross(self, enc):
        enc = np.ascontiguousarray(enc, np.float32)
        lib().or_state_prepare_cross(self.m._h, self._h, _p(enc), enc.shape[0])

    def forward(self, enc):
        enc = np.ascontiguousarray(enc, np.float32)
        out = np.empty(self.m.n_vocab, np.float32)
        if lib().or_forward(self.m._h, self._h, _p(enc), enc.shape[0], _p(out)) != 0:
            raise RuntimeError(lib().or_last_error().decode())
        return out


def conv1d(x, w, b, stride):
    """ml/conv.go:19-70 on x [in_c, T], w [out_c, in_c, k], b [out_c] -> [out_c, T']."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    in_c, t = x.shape
    out_c, _, k = w.shape
    tp = (t + 2 * (k // 2) - k) // stride + 1
    out = np.empty((out_c, tp), np.float32)
    lib().or_conv1d(_p(x), in_c, t, _p(w), _p(b), out_c, k, stride, _p(out))
    return out


def _tensor_array(tensors, keep):
    arr = (OrTensor * len(tensors))()
    for i, t in enumerate(tensors):
        name = t.name.encode()
        data = np.ascontiguousarray(t.data)
        keep += [name, data]
        arr[i].name, arr[i].type, arr[i].ndim = name, t.type, len(t.shape)
        for j, s in enumerate(t.shape):
            arr[i].shape[j] = s
        arr[i].data, arr[i].nbytes = data.ctypes.data, data.size
    return arr


class OracleEncoder:
    """or_encoder (model/encoder.go) over a tensor table."""

    def __init__(self, tensors, meta=None, dot_variant=1, threads=1):
        self._keep = []
        self._arr = _tensor_array(tensors, self._keep)
        m = OrEncMeta(**(meta or {}))
        self._h = lib().or_encoder_create(self._arr, len(tensors), C.byref(m), dot_variant, threads)
        if not self._h:
            raise RuntimeError(lib().or_last_error().decode())
        hp = np.zeros(5, np.int32)
        lib().or_encoder_hparams(self._h, _p(hp))
        self.n_mels, self.n_state, self.n_head, self.n_layer, self.n_ctx = (int(v) for v in hp)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().or_encoder_destroy(self._h)
            self._h = None

    def set_fast_exp(self, on):
        lib().or_encoder_set_fast_exp(self._h, int(on))

    def encode(self, mel):
        """mel [n_mels, T] -> encoder output [T', n_state] (T' = T / 2)."""
        mel = np.ascontiguousarray(mel, np.float32)
        nm, t = mel.shape
        out = np.empty((max(1, (min(t, 2 * self.n_ctx) + 1) // 2), self.n_state), np.float32)
        tp = lib().or_encode(self._h, _p(mel), nm, t, _p(out))
        if tp < 0:
            raise RuntimeError(lib().or_last_error().decode())
        return out[:tp]
