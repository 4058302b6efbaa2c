"""ctypes wrapper for the CPU oracle (fletcher_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker / CPU baseline, never by the
product package.  The oracle restates the reference CPU path
(internal/device/cpu_backend.go, internal/simd/simd.go,
internal/embeddings/model/bert.go) over OpenBLAS sgemm.
"""
from __future__ import annotations

import ctypes as C
import glob
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libfletcher_oracle.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")


def find_openblas() -> str:
    """scipy's bundled OpenBLAS (exports scipy_cblas_sgemm, LP64)."""
    env = os.environ.get("FLETCHER_ORACLE_BLAS")
    if env:
        return env
    import scipy
    cands = sorted(glob.glob(os.path.join(os.path.dirname(scipy.__file__) + ".libs",
                                          "libscipy_openblas*.so")))
    cands = [c for c in cands if "64_" not in os.path.basename(c)]
    if not cands:
        raise RuntimeError("no OpenBLAS found for the oracle")
    return cands[0]


class _Cfg(C.Structure):
    _fields_ = [("vocab_size", C.c_int32), ("hidden", C.c_int32), ("layers", C.c_int32),
                ("heads", C.c_int32), ("intermediate", C.c_int32), ("max_pos", C.c_int32),
                ("activation", C.c_int32), ("position", C.c_int32), ("rope_base", C.c_float),
                ("ln_eps", C.c_float), ("pool", C.c_int32), ("math", C.c_int32)]


_PP = C.POINTER(C.c_void_p)


class _Weights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("word_emb", "pos_emb", "type_emb", "emb_ln_g",
                                          "emb_ln_b")] + \
               [(n, _PP) for n in ("q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "o_b",
                                   "attn_ln_g", "attn_ln_b", "inter_w", "inter_b", "out_w",
                                   "out_b", "out_ln_g", "out_ln_b")] + \
               [(n, C.c_void_p) for n in ("pool_w", "pool_b")]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"oracle not built: {LIB_PATH} (run `make -C oracle`)")
    L = C.CDLL(str(LIB_PATH))
    if L.orc_blas_init(find_openblas().encode()) != 0:
        raise RuntimeError("oracle could not load OpenBLAS")
    L.orc_exp_fast.restype = C.c_float
    L.orc_exp_fast.argtypes = [C.c_float]
    L.orc_tanh_fast.restype = C.c_float
    L.orc_tanh_fast.argtypes = [C.c_float]
    L.orc_dot.restype = C.c_float
    L.orc_dot.argtypes = [_f32p, _f32p, C.c_int64]
    L.orc_f32_to_f16.restype = C.c_uint16
    L.orc_f32_to_f16.argtypes = [C.c_float]
    L.orc_f16_to_f32.restype = C.c_float
    L.orc_f16_to_f32.argtypes = [C.c_uint16]
    L.orc_gelu_fast.argtypes = [_f32p, C.c_int64]
    L.orc_softmax_fast.argtypes = [_f32p, C.c_int64]
    L.orc_add.argtypes = [_f32p, _f32p, C.c_int64]
    L.orc_scale.argtypes = [_f32p, C.c_int64, C.c_float]
    L.orc_add_bias.argtypes = [_f32p, C.c_int, C.c_int, _f32p]
    L.orc_tanh_inplace.argtypes = [_f32p, C.c_int64]
    L.orc_softmax_rows.argtypes = [_f32p, C.c_int, C.c_int]
    L.orc_layernorm.argtypes = [_f32p, C.c_int, C.c_int, _f32p, _f32p, C.c_float]
    L.orc_add_layernorm.argtypes = [_f32p, _f32p, C.c_int, C.c_int, _f32p, _f32p, C.c_float]
    L.orc_mul.argtypes = [_f32p, _f32p, C.c_int, C.c_int, C.c_int, _f32p, C.c_int, C.c_int,
                          C.c_int]
    L.orc_linear.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_int, C.c_void_p, _f32p]
    L.orc_linear_activation.argtypes = [_f32p, C.c_int, C.c_int, _f32p, C.c_int, C.c_void_p,
                                        C.c_int, _f32p]
    L.orc_gather.argtypes = [_f32p, C.c_int, C.c_int, _i64p, C.c_int, _f32p]
    L.orc_attention.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                C.c_float, _f32p]
    L.orc_attention_varlen.argtypes = [_f32p, _f32p, _f32p, _i64p, C.c_int, C.c_int, C.c_int,
                                       C.c_float, _f32p]
    L.orc_rope.argtypes = [_f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_double]
    L.orc_set_threads.argtypes = [C.c_int]
    L.orc_forward_batch.argtypes = [C.POINTER(_Cfg), C.POINTER(_Weights), _i64p, _i64p,
                                    C.c_int, _f32p, C.c_void_p]
    L.orc_forward_batch.restype = C.c_int
    _lib = L
    L.orc_set_threads(1)
    return L


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- simd.go ---------------------------------------------------------------
def exp_fast(x: float) -> float:
    return lib().orc_exp_fast(float(x))


def tanh_fast(x: float) -> float:
    return lib().orc_tanh_fast(float(x))


def exp_fast_vec(xs) -> np.ndarray:
    f = lib().orc_exp_fast
    return np.array([f(float(x)) for x in np.asarray(xs, np.float32)], np.float32)


def tanh_fast_vec(xs) -> np.ndarray:
    f = lib().orc_tanh_fast
    return np.array([f(float(x)) for x in np.asarray(xs, np.float32)], np.float32)


def gelu_fast(x) -> np.ndarray:
    a = _f32(x).copy()
    lib().orc_gelu_fast(a, a.size)
    return a


def softmax_fast(row) -> np.ndarray:
    a = _f32(row).copy()
    lib().orc_softmax_fast(a, a.size)
    return a


def dot(a, b) -> float:
    return lib().orc_dot(_f32(a), _f32(b), int(np.asarray(a).size))


# ---- utils.go --------------------------------------------------------------
def f32_to_f16_bits(x: float) -> int:
    return int(lib().orc_f32_to_f16(float(x)))


def f16_bits_to_f32(h: int) -> float:
    return float(lib().orc_f16_to_f32(int(h)))


# ---- cpu_backend.go --------------------------------------------------------
def add(t, other):
    a = _f32(t).copy()
    lib().orc_add(a, _f32(other), a.size)
    return a


def scale(t, v):
    a = _f32(t).copy()
    lib().orc_scale(a, a.size, float(v))
    return a


def add_bias(t, bias):
    a = _f32(t).copy()
    r, c = a.shape
    lib().orc_add_bias(a, r, c, _f32(bias))
    return a


def tanh(t):
    a = _f32(t).copy()
    lib().orc_tanh_inplace(a, a.size)
    return a


def softmax_rows(t):
    a = _f32(t).copy()
    r, c = a.shape
    lib().orc_softmax_rows(a, r, c)
    return a


def layernorm(t, gamma, beta, eps):
    a = _f32(t).copy()
    r, c = a.shape
    lib().orc_layernorm(a, r, c, _f32(gamma), _f32(beta), float(eps))
    return a


def add_layernorm(t, residual, gamma, beta, eps):
    a = _f32(t).copy()
    r, c = a.shape
    lib().orc_add_layernorm(a, _f32(residual), r, c, _f32(gamma), _f32(beta), float(eps))
    return a


def mul(a, b, trans_a=False, trans_b=False):
    a = _f32(a)
    b = _f32(b)
    m = a.shape[1] if trans_a else a.shape[0]
    n = b.shape[0] if trans_b else b.shape[1]
    c = np.zeros((m, n), np.float32)
    lib().orc_mul(c, a, a.shape[0], a.shape[1], int(trans_a), b, b.shape[0], b.shape[1],
                  int(trans_b))
    return c


def linear(x, w, bias=None):
    x = _f32(x)
    w = _f32(w)
    out = np.zeros((x.shape[0], w.shape[1]), np.float32)
    bkeep = _f32(bias) if bias is not None else None
    lib().orc_linear(x, x.shape[0], x.shape[1], w, w.shape[1],
                     bkeep.ctypes.data if bkeep is not None else None, out)
    return out


def linear_activation(x, w, bias, act):
    x = _f32(x)
    w = _f32(w)
    n = w.shape[1]
    cols = n // 2 if act == 4 else n
    out = np.zeros((x.shape[0], cols), np.float32)
    bkeep = _f32(bias) if bias is not None else None
    lib().orc_linear_activation(x, x.shape[0], x.shape[1], w, n,
                                bkeep.ctypes.data if bkeep is not None else None, int(act), out)
    return out


def gather(table, idx):
    table = _f32(table)
    idx = np.ascontiguousarray(idx, np.int64)
    out = np.zeros((idx.size, table.shape[1]), np.float32)
    lib().orc_gather(table, table.shape[0], table.shape[1], idx, idx.size, out)
    return out


def attention(q, k, v, batch, seq, heads, scale_):
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros_like(q)
    lib().orc_attention(q, k, v, batch, seq, heads, q.shape[1], float(scale_), out)
    return out


def attention_varlen(q, k, v, lengths, heads, scale_):
    q, k, v = _f32(q), _f32(k), _f32(v)
    lengths = np.ascontiguousarray(lengths, np.int64)
    out = np.zeros_like(q)
    lib().orc_attention_varlen(q, k, v, lengths, lengths.size, heads, q.shape[1],
                               float(scale_), out)
    return out


def rope(t, batch, seq, heads, head_dim, base=10000.0):
    a = _f32(t).copy()
    lib().orc_rope(a, batch, seq, heads, head_dim, float(base))
    return a


# ---- bert.go ---------------------------------------------------------------
def forward(cfg, weights: dict, ids, lengths, math_mode: int = 0, pool: int | None = None,
            return_hidden: bool = False):
    """BertModel.ForwardBatch + pooling on the CPU oracle.  `cfg` is a
    synth.ModelConfig; `weights` the dict from synth.make_weights."""
    L = lib()
    ids = np.ascontiguousarray(ids, np.int64)
    lengths = np.ascontiguousarray(lengths, np.int64)
    c = _Cfg(cfg.vocab_size, cfg.hidden, cfg.layers, cfg.heads, cfg.intermediate, cfg.max_pos,
             cfg.activation, cfg.position, cfg.rope_base, cfg.ln_eps,
             cfg.pool if pool is None else pool, math_mode)
    keep = []

    def ptr(name):
        a = weights.get(name)
        if a is None:
            return None
        a = _f32(a)
        keep.append(a)
        return a.ctypes.data

    def arr(field):
        names = [f"{field}.{l}" for l in range(cfg.layers)]
        if names[0] not in weights:
            return None
        vals = (C.c_void_p * cfg.layers)(*[ptr(n) for n in names])
        keep.append(vals)
        return C.cast(vals, _PP)

    w = _Weights()
    for n in ("word_emb", "pos_emb", "type_emb", "emb_ln_g", "emb_ln_b", "pool_w", "pool_b"):
        setattr(w, n, ptr(n))
    for f in ("q_w", "q_b", "k_w", "k_b", "v_w", "v_b", "o_w", "o_b", "attn_ln_g", "attn_ln_b",
              "inter_w", "inter_b", "out_w", "out_b", "out_ln_g", "out_ln_b"):
        setattr(w, f, arr(f))
    out = np.zeros((lengths.size, cfg.hidden), np.float32)
    hidden = np.zeros((int(lengths.sum()), cfg.hidden), np.float32) if return_hidden else None
    rc = L.orc_forward_batch(C.byref(c), C.byref(w), ids, lengths, lengths.size, out,
                             hidden.ctypes.data if hidden is not None else None)
    if rc != 0:
        raise RuntimeError(f"orc_forward_batch failed: {rc}")
    return (out, hidden) if return_hidden else out
