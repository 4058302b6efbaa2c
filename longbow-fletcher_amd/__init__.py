"""Python host binding of the gfx950 encoder-forward backend (ctypes over
include/fletcher_hip.h).

Mirrors the reference's device interface for this path
(internal/device/device.go:5-162): a `Context` is a Backend (device, stream,
buffers), the op methods are the Tensor methods, and `Model` is
BertModel.ForwardBatch (internal/embeddings/model/bert.go:149-169).
Failures raise FletcherError carrying the library's status code and message,
where the reference panics.

The product path is libfletcher_hip.so only: if the library is missing this
module raises on use; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import re

import numpy as np

from . import synth  # noqa: F401  (re-exported for callers)

PKG = pathlib.Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libfletcher_hip.so"
HEADER = PKG.parent / "include" / "fletcher_hip.h"

OK, ERR_INVALID, ERR_HIP, ERR_OOM, ERR_UNSUPPORTED, ERR_IO = 0, 1, 2, 3, 4, 5
F32, F16, BF16 = 0, 1, 2
ACT_IDENTITY, ACT_GELU, ACT_TANH, ACT_SOFTMAX, ACT_SWIGLU = 0, 1, 2, 3, 4
MATH_REFERENCE, MATH_EXACT = 0, 1
ROUND_NEAREST, ROUND_TRUNCATE = 0, 1
W_IN_OUT, W_OUT_IN = 0, 1
POOL_CLS_TANH, POOL_MEAN, POOL_MEAN_L2 = 0, 1, 2
POS_ABSOLUTE, POS_ROPE = 0, 1
PROF_CLASSES = ("embed", "qkv_gemm", "attention", "o_gemm", "add_layernorm", "ffn_up_gemm",
                "ffn_down_gemm", "pool")

_NP = {F32: np.float32, F16: np.float16}
_ESZ = {F32: 4, F16: 2, BF16: 2}


class FletcherError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class ModelConfigC(C.Structure):
    _fields_ = [("vocab_size", C.c_int32), ("hidden", C.c_int32), ("layers", C.c_int32),
                ("heads", C.c_int32), ("intermediate", C.c_int32), ("max_pos", C.c_int32),
                ("activation", C.c_int32), ("position", C.c_int32), ("rope_base", C.c_float),
                ("ln_eps", C.c_float), ("dtype", C.c_int32), ("math", C.c_int32),
                ("pool", C.c_int32), ("has_bias", C.c_int32)]


_vp, _i, _i64, _f, _cp = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_char_p
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")

_SIGS = {
    "fl_last_error": ([], _cp),
    "fl_version": ([], _cp),
    "fl_device_count": ([C.POINTER(_i)], _i),
    "fl_init": ([_i, C.POINTER(_vp)], _i),
    "fl_free_context": ([_vp], _i),
    "fl_set_device": ([_vp, _i], _i),
    "fl_synchronize": ([_vp], _i),
    "fl_vram_usage": ([_vp, C.POINTER(_i64), C.POINTER(_i64)], _i),
    "fl_get_stream": ([_vp, C.POINTER(_vp)], _i),
    "fl_alloc": ([_vp, _i64, C.POINTER(_vp)], _i),
    "fl_alloc_uninit": ([_vp, _i64, C.POINTER(_vp)], _i),
    "fl_free": ([_vp, _vp], _i),
    "fl_pool_stats": ([_vp, C.POINTER(_i64)], _i),
    "fl_pool_trim": ([_vp], _i),
    "fl_buffer_written": ([_vp, _vp], _i),
    "fl_copy_to_device": ([_vp, _vp, _vp, _i64], _i),
    "fl_copy_to_host": ([_vp, _vp, _vp, _i64], _i),
    "fl_copy_device": ([_vp, _vp, _vp, _i64], _i),
    "fl_memset": ([_vp, _vp, _i, _i64], _i),
    "fl_upload_f32": ([_vp, _vp, _i, _vp, _i64, _i], _i),
    "fl_download_f32": ([_vp, _vp, _vp, _i, _i64], _i),
    "fl_gemm": ([_vp, _i, _i, _i, _i, _i, _i, _f, _vp, _i, _vp, _i, _vp, _i], _i),
    "fl_linear": ([_vp, _i, _vp, _i, _i, _i, _vp, _i, _i, _vp, _i, _i, _vp], _i),
    "fl_add": ([_vp, _i, _vp, _i, _vp, _i64], _i),
    "fl_add_scalar": ([_vp, _i, _vp, _i64, _f], _i),
    "fl_scale": ([_vp, _i, _vp, _i64, _f], _i),
    "fl_add_bias": ([_vp, _i, _vp, _i, _i, _vp], _i),
    "fl_activation": ([_vp, _i, _vp, _i, _i, _i, _i], _i),
    "fl_layernorm": ([_vp, _i, _vp, _i, _i, _vp, _vp, _f], _i),
    "fl_add_layernorm": ([_vp, _i, _vp, _i, _vp, _i, _i, _vp, _vp, _f], _i),
    "fl_gather_rows": ([_vp, _i, _vp, _i, _i, _vp, _i, _vp], _i),
    "fl_rope": ([_vp, _i, _vp, _i, _i, _i, _i, _f], _i),
    "fl_rope_varlen": ([_vp, _i, _vp, _vp, _i, _i, _i, _f], _i),
    "fl_attention": ([_vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i], _i),
    "fl_attention_varlen": ([_vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _i], _i),
    "fl_cast": ([_vp, _vp, _i, _vp, _i, _i64], _i),
    "fl_has_nan": ([_vp, _vp, _i, _i64, C.POINTER(_i)], _i),
    "fl_slice": ([_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp], _i),
    "fl_mean_pool": ([_vp, _i, _vp, _i, _vp, _i, _i, _vp], _i),
    "fl_mean_pool_noalloc": ([_vp, _i, _vp, _i, _vp, _i, _i, _vp], _i),
    "fl_model_create": ([_vp, C.POINTER(ModelConfigC), C.POINTER(_vp)], _i),
    "fl_model_free": ([_vp], _i),
    "fl_model_set_weight": ([_vp, _cp, _vp, _i64], _i),
    "fl_model_load_raw": ([_vp, _cp], _i),
    "fl_model_embed": ([_vp, _vp, _vp, _i, _i, _i64, _vp, _vp, C.POINTER(_i)], _i),
    "fl_model_load_safetensors": ([_vp, _cp], _i),
    "fl_model_forward": ([_vp, _vp, _vp, _i, _vp], _i),
    "fl_model_forward_ex": ([_vp, _vp, _vp, _i, _i, _vp], _i),
    "fl_model_embed_ex": ([_vp, _vp, _vp, _i, _i, _i64, _i, _vp, _vp, C.POINTER(_i)], _i),
    "fl_model_forward_padded": ([_vp, _vp, _vp, _i, _i, _vp], _i),
    "fl_model_forward_device": ([_vp, _vp, _vp, _i, _vp], _i),
    "fl_model_status": ([_vp, C.POINTER(_i), C.POINTER(_i)], _i),
    "fl_model_last_hidden": ([_vp, _vp, _i64], _i),
    "fl_model_set_profiling": ([_vp, _i], _i),
    "fl_model_profile_read": ([_vp, C.POINTER(C.c_double), C.POINTER(_i64)], _i),
}

_lib = None


def header_symbols() -> list[str]:
    """Entry points declared in include/fletcher_hip.h."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(fl_\w+)\s*\(", text, re.M)))


def lib():
    """Loads libfletcher_hip.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FletcherError(ERR_UNSUPPORTED,
                            f"{LIB_PATH} missing: build it with longbow-fletcher_amd/build.py")
    L = C.CDLL(str(LIB_PATH))
    for name, (args, res) in _SIGS.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != OK:
        raise FletcherError(rc, lib().fl_last_error().decode(errors="replace"))


def device_count() -> int:
    n = C.c_int(0)
    check(lib().fl_device_count(C.byref(n)))
    return n.value


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    return int(x)


class DeviceArray:
    """A device buffer of `shape` in storage dtype F32 / F16 / BF16 (a Tensor)."""

    def __init__(self, ctx: "Context", ptr: int, shape, dtype: int, owned: bool = True):
        self.ctx, self.ptr, self.shape, self.dtype, self.owned = ctx, ptr, tuple(shape), dtype, owned

    @property
    def size(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.size * _ESZ[self.dtype]

    def numpy(self) -> np.ndarray:
        """Tensor.ToHost: values as float32."""
        out = np.empty(self.size, np.float32)
        check(lib().fl_download_f32(self.ctx.h, out.ctypes.data, self.ptr, self.dtype, self.size))
        return out.reshape(self.shape)

    def raw(self) -> np.ndarray:
        """The stored bytes (uint16 for 16-bit types)."""
        dt = np.float32 if self.dtype == F32 else np.uint16
        out = np.empty(self.size, dt)
        check(lib().fl_copy_to_host(self.ctx.h, out.ctypes.data, self.ptr, self.nbytes))
        return out.reshape(self.shape)

    def rows_view(self, r0: int, r1: int) -> "DeviceArray":
        """Rows [r0, r1) of a 2-D tensor as a non-owning view (Tensor.Slice of
        all columns, metal_darwin.go:487-521): writes through it land here."""
        rows, cols = self.shape
        if not 0 <= r0 < r1 <= rows:
            raise FletcherError(ERR_INVALID, "Slice: invalid dimensions")
        return DeviceArray(self.ctx, self.ptr + r0 * cols * _ESZ[self.dtype], (r1 - r0, cols),
                           self.dtype, owned=False)

    def free(self):
        if self.owned and self.ptr:
            check(lib().fl_free(self.ctx.h, self.ptr))
        self.ptr = 0


class Context:
    """Backend (device.go:137-162) on one GPU: stream, buffers, ops."""

    def __init__(self, device: int = 0):
        h = C.c_void_p()
        check(lib().fl_init(device, C.byref(h)))
        self.h = h.value

    # -- Backend --------------------------------------------------------
    def close(self):
        if self.h:
            check(lib().fl_free_context(self.h))
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def synchronize(self):
        check(lib().fl_synchronize(self.h))

    def vram_usage(self):
        a, t = C.c_int64(), C.c_int64()
        check(lib().fl_vram_usage(self.h, C.byref(a), C.byref(t)))
        return a.value, t.value

    def pool_stats(self) -> dict:
        """The buffer cache's counters (hits, misses, cached bytes / buffers,
        packed-weight bytes, buffers in use)."""
        st = (C.c_int64 * 6)()
        check(lib().fl_pool_stats(self.h, st))
        return dict(zip(("hits", "misses", "cached_bytes", "cached_buffers", "packed_bytes",
                         "live_buffers"), list(st)))

    def pool_trim(self):
        check(lib().fl_pool_trim(self.h))

    def buffer_written(self, t: "DeviceArray"):
        check(lib().fl_buffer_written(self.h, t.ptr))

    def stream(self) -> int:
        s = C.c_void_p()
        check(lib().fl_get_stream(self.h, C.byref(s)))
        return s.value or 0

    # -- buffers --------------------------------------------------------
    def empty(self, shape, dtype: int = F32) -> DeviceArray:
        """Backend.GetTensor: zero-filled."""
        n = int(np.prod(shape)) if len(shape) else 1
        p = C.c_void_p()
        check(lib().fl_alloc(self.h, n * _ESZ[dtype], C.byref(p)))
        return DeviceArray(self, p.value, shape, dtype)

    def result(self, shape, dtype: int = F32) -> DeviceArray:
        """The result tensor of a producing op, which writes it whole: not
        zero-filled (fl_alloc_uninit)."""
        n = int(np.prod(shape)) if len(shape) else 1
        p = C.c_void_p()
        check(lib().fl_alloc_uninit(self.h, n * _ESZ[dtype], C.byref(p)))
        return DeviceArray(self, p.value, shape, dtype)

    def tensor(self, data, dtype: int = F32, rounding: int = ROUND_NEAREST) -> DeviceArray:
        """Backend.NewTensorWithType + CopyFromFloat32."""
        a = np.ascontiguousarray(data, dtype=np.float32)
        t = self.result(a.shape, dtype)
        check(lib().fl_upload_f32(self.h, t.ptr, dtype, a.ctypes.data, a.size, rounding))
        return t

    def int32(self, data) -> DeviceArray:
        a = np.ascontiguousarray(data, dtype=np.int32)
        t = self.result(a.shape, F32)
        check(lib().fl_copy_to_device(self.h, t.ptr, a.ctypes.data, a.nbytes))
        return t

    # -- Tensor ops -----------------------------------------------------
    def gemm(self, a: DeviceArray, b: DeviceArray, trans_a=False, trans_b=False, alpha=1.0):
        m = a.shape[1] if trans_a else a.shape[0]
        k = a.shape[0] if trans_a else a.shape[1]
        n = b.shape[0] if trans_b else b.shape[1]
        c = self.result((m, n), a.dtype)
        check(lib().fl_gemm(self.h, a.dtype, int(trans_a), int(trans_b), m, n, k, alpha, a.ptr,
                            a.shape[1], b.ptr, b.shape[1], c.ptr, n))
        return c

    def linear(self, x: DeviceArray, w: DeviceArray, bias=None, act=ACT_IDENTITY,
               math=MATH_REFERENCE, w_layout=W_IN_OUT):
        """out = act(x W + bias); the result has W's storage type and x is
        converted to it (Linear on the reference's Metal backend)."""
        rows, k = x.shape
        n = w.shape[1] if w_layout == W_IN_OUT else w.shape[0]
        out = self.result((rows, n // 2 if act == ACT_SWIGLU else n), w.dtype)
        check(lib().fl_linear(self.h, x.dtype, x.ptr, rows, k, w.dtype, w.ptr, w_layout, n,
                              _ptr(bias), act, math, out.ptr))
        return out

    def add(self, t: DeviceArray, o: DeviceArray):
        """t += o (o converted to t's storage type)."""
        check(lib().fl_add(self.h, t.dtype, t.ptr, o.dtype, o.ptr, t.size))

    def add_scalar(self, t: DeviceArray, v: float):
        check(lib().fl_add_scalar(self.h, t.dtype, t.ptr, t.size, v))

    def scale(self, t: DeviceArray, v: float):
        check(lib().fl_scale(self.h, t.dtype, t.ptr, t.size, v))

    def add_bias(self, t: DeviceArray, bias: DeviceArray):
        check(lib().fl_add_bias(self.h, t.dtype, t.ptr, t.shape[0], t.shape[1], bias.ptr))

    def activation(self, t: DeviceArray, act: int, math=MATH_REFERENCE):
        check(lib().fl_activation(self.h, t.dtype, t.ptr, t.shape[0], t.shape[1], act, math))

    def layernorm(self, t: DeviceArray, gamma: DeviceArray, beta: DeviceArray, eps: float):
        check(lib().fl_layernorm(self.h, t.dtype, t.ptr, t.shape[0], t.shape[1], gamma.ptr,
                                 beta.ptr, eps))

    def add_layernorm(self, t, residual, gamma, beta, eps):
        """t = LayerNorm(t + residual), the residual converted to t's type."""
        check(lib().fl_add_layernorm(self.h, t.dtype, t.ptr, residual.dtype, residual.ptr,
                                     t.shape[0], t.shape[1], gamma.ptr, beta.ptr, eps))

    def gather(self, table: DeviceArray, idx) -> DeviceArray:
        idx = np.ascontiguousarray(idx, np.int64)
        out = self.result((idx.size, table.shape[1]), table.dtype)
        check(lib().fl_gather_rows(self.h, table.dtype, table.ptr, table.shape[0],
                                   table.shape[1], idx.ctypes.data, idx.size, out.ptr))
        return out

    def rope(self, t: DeviceArray, batch, seq, heads, head_dim, base=10000.0):
        check(lib().fl_rope(self.h, t.dtype, t.ptr, batch, seq, heads, head_dim, base))

    def rope_varlen(self, t: DeviceArray, lengths, heads, head_dim, base=10000.0):
        lengths = np.ascontiguousarray(lengths, np.int64)
        check(lib().fl_rope_varlen(self.h, t.dtype, t.ptr, lengths.ctypes.data, lengths.size,
                                   heads, head_dim, base))

    def attention(self, q, k, v, batch, seq, heads, scale, math=MATH_REFERENCE):
        out = self.result(q.shape, q.dtype)
        check(lib().fl_attention(self.h, q.dtype, q.ptr, k.ptr, v.ptr, out.ptr, batch, seq, heads,
                                 q.shape[1], scale, math))
        return out

    def attention_varlen(self, q, k, v, lengths, heads, scale, math=MATH_REFERENCE):
        lengths = np.ascontiguousarray(lengths, np.int64)
        out = self.result(q.shape, q.dtype)
        check(lib().fl_attention_varlen(self.h, q.dtype, q.ptr, k.ptr, v.ptr, out.ptr,
                                        lengths.ctypes.data, lengths.size, heads, q.shape[1],
                                        scale, math))
        return out

    def cast(self, t: DeviceArray, dtype: int) -> DeviceArray:
        out = self.result(t.shape, dtype)
        check(lib().fl_cast(self.h, t.ptr, t.dtype, out.ptr, dtype, t.size))
        return out

    def has_nan(self, t: DeviceArray) -> bool:
        r = C.c_int(0)
        check(lib().fl_has_nan(self.h, t.ptr, t.dtype, t.size, C.byref(r)))
        return bool(r.value)

    def slice(self, t: DeviceArray, r0, r1, c0, c1) -> DeviceArray:
        out = self.result((max(r1 - r0, 0), max(c1 - c0, 0)), t.dtype)
        check(lib().fl_slice(self.h, t.dtype, t.ptr, t.shape[0], t.shape[1], r0, r1, c0, c1,
                             out.ptr))
        return out

    def mean_pool(self, hidden: DeviceArray, lengths, l2=True, out: DeviceArray = None,
                  noalloc: bool = False) -> DeviceArray:
        """Masked mean-pool (+L2) of packed rows.  noalloc=True calls
        fl_mean_pool_noalloc, which allocates nothing on the device (out must
        then be given)."""
        lengths = np.ascontiguousarray(lengths, np.int64)
        if out is None:
            out = self.result((lengths.size, hidden.shape[1]), F32)
        f = lib().fl_mean_pool_noalloc if noalloc else lib().fl_mean_pool
        check(f(self.h, hidden.dtype, hidden.ptr, hidden.shape[1], lengths.ctypes.data,
                lengths.size, int(l2), out.ptr))
        return out


def plan_batches(lengths, max_seqs: int = 512, max_tokens: int = 16384):
    """The (first sequence, count) batches of fl_model_embed's plan: the
    batching loop of runInferenceOnDevice (embeddings.go:704-731).  The
    library computes consecutive batches of the plan together, in forwards
    of up to 65536 tokens; the vectors and per-batch NaN flags are those of
    one forward per batch."""
    plan, i, n = [], 0, len(lengths)
    while i < n:
        size, tokens = 0, 0
        for j in range(i, n):
            if size >= max_seqs or (tokens + int(lengths[j]) > max_tokens and size > 0):
                break
            tokens += int(lengths[j])
            size += 1
        size = max(size, 1)
        plan.append((i, size))
        i += size
    return plan


class Model:
    """BertModel on the HIP backend (bert.go:77-169)."""

    def __init__(self, ctx: Context, cfg, dtype: int = F16, math: int = MATH_EXACT,
                 pool: int | None = None):
        self.ctx, self.cfg, self.dtype = ctx, cfg, dtype
        c = ModelConfigC(cfg.vocab_size, cfg.hidden, cfg.layers, cfg.heads, cfg.intermediate,
                         cfg.max_pos, cfg.activation, cfg.position, cfg.rope_base, cfg.ln_eps,
                         dtype, math, cfg.pool if pool is None else pool, int(cfg.has_bias))
        h = C.c_void_p()
        check(lib().fl_model_create(ctx.h, C.byref(c), C.byref(h)))
        self.h = h.value

    def close(self):
        if self.h:
            check(lib().fl_model_free(self.h))
            self.h = None

    def set_weight(self, name: str, data) -> None:
        a = np.ascontiguousarray(data, np.float32)
        check(lib().fl_model_set_weight(self.h, name.encode(), a.ctypes.data, a.size))

    def load(self, weights: dict) -> "Model":
        for name, arr in weights.items():
            self.set_weight(name, arr)
        return self

    def load_raw(self, path) -> "Model":
        """Loader.LoadFromRawBinary (weights/loader.go:29-90)."""
        check(lib().fl_model_load_raw(self.h, os.fsencode(path)))
        return self

    def load_safetensors(self, path) -> "Model":
        """Loader.LoadFromSafeTensors (weights/loader.go:155-237)."""
        check(lib().fl_model_load_safetensors(self.h, os.fsencode(path)))
        return self

    def forward(self, ids, lengths, out_dtype: int = F32) -> np.ndarray:
        """Pooled vectors, float32 or (out_dtype=F16) float16 converted on the
        device (processOutput's fp16 transport, embeddings.go:256-286)."""
        ids = np.ascontiguousarray(ids, np.int64)
        lengths = np.ascontiguousarray(lengths, np.int64)
        out = np.zeros((lengths.size, self.cfg.hidden), _NP.get(out_dtype, np.uint16))
        if out_dtype == F32:
            check(lib().fl_model_forward(self.h, ids.ctypes.data, lengths.ctypes.data,
                                         lengths.size, out.ctypes.data))
        else:
            check(lib().fl_model_forward_ex(self.h, ids.ctypes.data, lengths.ctypes.data,
                                            lengths.size, out_dtype, out.ctypes.data))
        return out

    def embed(self, ids, lengths, max_seqs: int = 512, max_tokens: int = 16384,
              out_dtype: int = F32):
        """All sequences through token-budget batches with overlapped copies
        (runInferenceOnDevice, embeddings.go:690-775).  Returns (pooled
        [nseq, hidden] float32 or float16, per-sequence NaN flag of its batch,
        batch count)."""
        ids = np.ascontiguousarray(ids, np.int64)
        lengths = np.ascontiguousarray(lengths, np.int64)
        out = np.zeros((lengths.size, self.cfg.hidden), _NP.get(out_dtype, np.uint16))
        nan = np.zeros(lengths.size, np.int32)
        nb = C.c_int()
        check(lib().fl_model_embed_ex(self.h, ids.ctypes.data, lengths.ctypes.data, lengths.size,
                                      int(max_seqs), int(max_tokens), out_dtype, out.ctypes.data,
                                      nan.ctypes.data, C.byref(nb)))
        return out, nan.astype(bool), nb.value

    def forward_padded(self, ids, mask) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int64)
        mask = np.ascontiguousarray(mask, np.int64)
        b, s = ids.shape
        out = np.zeros((b, self.cfg.hidden), np.float32)
        check(lib().fl_model_forward_padded(self.h, ids.ctypes.data, mask.ctypes.data, b, s,
                                            out.ctypes.data))
        return out

    def forward_device(self, d_ids: DeviceArray, lengths, d_out: DeviceArray) -> None:
        lengths = np.ascontiguousarray(lengths, np.int64)
        check(lib().fl_model_forward_device(self.h, d_ids.ptr, lengths.ctypes.data, lengths.size,
                                            d_out.ptr))

    def status(self):
        a, b = C.c_int(), C.c_int()
        check(lib().fl_model_status(self.h, C.byref(a), C.byref(b)))
        return bool(a.value), bool(b.value)

    def last_hidden(self, total_tokens: int) -> np.ndarray:
        out = np.zeros((total_tokens, self.cfg.hidden), np.float32)
        check(lib().fl_model_last_hidden(self.h, out.ctypes.data, out.size))
        return out

    def set_profiling(self, on: bool) -> None:
        check(lib().fl_model_set_profiling(self.h, int(on)))

    def profile(self) -> dict:
        ms = (C.c_double * len(PROF_CLASSES))()
        cnt = (C.c_int64 * len(PROF_CLASSES))()
        check(lib().fl_model_profile_read(self.h, ms, cnt))
        return {n: (ms[i], cnt[i]) for i, n in enumerate(PROF_CLASSES)}
