"""The reference's device interface on this backend, method for method.

`RocmBackend` is `device.Backend` and `RocmTensor` is `device.Tensor`
(internal/device/device.go:5-162), written over the C ABI exactly as the Go
binding `internal/device/rocm_linux.go` writes them over cgo:
the same entry points, the same arguments, the same storage-type rules.
Method names keep Go's spelling so that code written against the interface
(bert.go, replayed by perop.py) reads the same here.

Storage-type rules (the reference's Metal backend, the GPU backend the model
code was written for):
  * NewTensor / GetTensor use the backend's type (Float16 for an fp16
    backend, metal_darwin.go:92-98);
  * Linear / LinearActivation: the result takes the weight's type and the
    input is converted to it (metal_darwin.go:806-829, 887-903);
  * Add / AddLayerNorm convert the other operand to the receiver's type
    (:603-619, 798-804); Mul computes in the receiver's type (:557-601);
  * Slice of all columns is a non-owning view (:487-521); other slices and
    Cast are copies (:522-541, 1178-1241); Copy needs equal types (:448-485).
Failures raise FletcherError where the Go binding panics.
"""
from __future__ import annotations

import ctypes as C
import math as _math

import numpy as np

from . import (ACT_GELU, ACT_IDENTITY, ACT_SOFTMAX, ACT_SWIGLU, ACT_TANH, ERR_INVALID, F16, F32,
               MATH_EXACT, MATH_REFERENCE, POOL_MEAN_L2, ROUND_NEAREST, W_IN_OUT, W_OUT_IN,
               FletcherError, check, lib)

Float32, Float16 = F32, F16
ActivationIdentity, ActivationGELU, ActivationTanh = ACT_IDENTITY, ACT_GELU, ACT_TANH
ActivationSoftmax, ActivationSwiGLU = ACT_SOFTMAX, ACT_SWIGLU

_ESZ = {0: 4, 1: 2, 2: 2}


def _esz(dt: int) -> int:
    return _ESZ[dt]


class RocmBackend:
    """device.Backend (device.go:137-162) on one GPU.

    dtype: storage type of NewTensor (Float32 or Float16).  math: the
    library's math mode for the fused ops; the binding uses the reference's
    fast-math formulas (MATH_REFERENCE) for an fp32 backend, so results match
    the CPU path to ~1e-6, and hardware exp2 with the flash kernels
    (MATH_EXACT) for a 16-bit one.  rope_base: ApplyRoPE's base, which the
    reference hard-codes to 10000 (cpu_backend.go:790)."""

    def __init__(self, device: int = 0, dtype: int = Float32, math: int | None = None,
                 rope_base: float = 10000.0):
        h = C.c_void_p()
        check(lib().fl_init(device, C.byref(h)))
        self.ctx = h.value
        self.dtype = dtype
        self.math = (MATH_REFERENCE if dtype == Float32 else MATH_EXACT) if math is None else math
        self.rope_base = float(rope_base)

    def close(self):
        if self.ctx:
            check(lib().fl_free_context(self.ctx))
            self.ctx = None

    def Name(self) -> str:
        return "ROCm-gfx950"

    def Synchronize(self):
        check(lib().fl_synchronize(self.ctx))

    def DeviceCount(self) -> int:
        n = C.c_int()
        check(lib().fl_device_count(C.byref(n)))
        return n.value

    def SetDevice(self, i: int):
        check(lib().fl_set_device(self.ctx, i))

    def GetVRAMUsage(self):
        a, t = C.c_int64(), C.c_int64()
        check(lib().fl_vram_usage(self.ctx, C.byref(a), C.byref(t)))
        return a.value, t.value

    # GetTensor / NewTensor without data hand out zeros (fl_alloc); tensors
    # written whole right away use fl_alloc_uninit.
    def _alloc(self, r: int, c: int, dt: int, zero: bool) -> "RocmTensor":
        p = C.c_void_p()
        f = lib().fl_alloc if zero else lib().fl_alloc_uninit
        check(f(self.ctx, r * c * _esz(dt), C.byref(p)))
        return RocmTensor(self, p.value, r, c, dt, owner=True)

    def _result(self, r: int, c: int, dt: int) -> "RocmTensor":
        return self._alloc(r, c, dt, False)

    def NewTensorWithType(self, r: int, c: int, dt: int, data=None) -> "RocmTensor":
        t = self._alloc(r, c, dt, data is None)
        if data is not None:
            t.CopyFromFloat32(data)
        return t

    def NewTensor(self, r: int, c: int, data=None) -> "RocmTensor":
        return self.NewTensorWithType(r, c, self.dtype, data)

    def GetTensor(self, r: int, c: int) -> "RocmTensor":
        return self.NewTensor(r, c, None)

    def PutTensor(self, t: "RocmTensor"):
        """Returns the buffer to the library's cache at once (fl_free does not
        wait for the device); views and tensors already put back are ignored."""
        if not isinstance(t, RocmTensor) or not t.owner or not t.ptr:
            return
        check(lib().fl_free(self.ctx, t.ptr))
        t.ptr = 0


class RocmTensor:
    """device.Tensor (device.go:5-117): a 2-D row-major device buffer, or a
    view into one (a transpose flag, or a row range)."""

    def __init__(self, b: RocmBackend, ptr: int, rows: int, cols: int, dt: int,
                 trans: bool = False, owner: bool = False):
        self.b, self.ptr, self.rows, self.cols, self.dt = b, ptr, rows, cols, dt
        self.trans, self.owner = trans, owner

    def __del__(self):
        # The Go binding's finalizer (runtime.SetFinalizer): a tensor never
        # put back is returned when it becomes unreachable.
        try:
            if self.owner and self.ptr and self.b.ctx:
                lib().fl_free(self.b.ctx, self.ptr)
        except Exception:
            pass

    # -- shape / host access ----------------------------------------------
    def Dims(self):
        return (self.cols, self.rows) if self.trans else (self.rows, self.cols)

    def DataType(self) -> int:
        return self.dt

    def Data(self):
        return None  # device resident

    def T(self) -> "RocmTensor":
        return RocmTensor(self.b, self.ptr, self.rows, self.cols, self.dt, not self.trans, False)

    def _index(self, i: int, j: int) -> int:
        r, c = self.Dims()
        if not (0 <= i < r and 0 <= j < c):
            raise FletcherError(ERR_INVALID, "Index out of bounds")
        return j * self.cols + i if self.trans else i * self.cols + j

    def At(self, i: int, j: int) -> float:
        out = np.zeros(1, np.float32)
        check(lib().fl_download_f32(self.b.ctx, out.ctypes.data,
                                    self.ptr + self._index(i, j) * _esz(self.dt), self.dt, 1))
        return float(out[0])

    def Set(self, i: int, j: int, v: float):
        a = np.array([v], np.float32)
        check(lib().fl_upload_f32(self.b.ctx, self.ptr + self._index(i, j) * _esz(self.dt),
                                  self.dt, a.ctypes.data, 1, ROUND_NEAREST))

    def CopyFromFloat32(self, data):
        a = np.ascontiguousarray(data, np.float32).ravel()
        if a.size != self.rows * self.cols:
            raise FletcherError(ERR_INVALID, "CopyFromFloat32: size mismatch")
        check(lib().fl_upload_f32(self.b.ctx, self.ptr, self.dt, a.ctypes.data, a.size,
                                  ROUND_NEAREST))

    def ToHost(self) -> np.ndarray:
        out = np.empty(self.rows * self.cols, np.float32)
        check(lib().fl_download_f32(self.b.ctx, out.ctypes.data, self.ptr, self.dt, out.size))
        if self.trans:
            return np.ascontiguousarray(out.reshape(self.rows, self.cols).T).ravel()
        return out

    def ExtractToFlat(self, dst: np.ndarray, start: int):
        h = self.ToHost()
        dst[start:start + h.size] = h

    def ExtractTo(self, dst: list, start: int):
        r, c = self.Dims()
        h = self.ToHost().reshape(r, c)
        for i in range(r):
            dst[start + i] = h[i].copy()

    def ExtractBytes(self) -> bytes:
        n = self.rows * self.cols * _esz(self.dt)
        out = np.empty(n, np.uint8)
        check(lib().fl_copy_to_host(self.b.ctx, out.ctypes.data, self.ptr, n))
        return out.tobytes()

    def HasNaN(self):
        r = C.c_int()
        check(lib().fl_has_nan(self.b.ctx, self.ptr, self.dt, self.rows * self.cols, C.byref(r)))
        return r.value != 0, None

    # -- copies, views, casts -----------------------------------------------
    def Copy(self, frm: "RocmTensor"):
        if frm.dt != self.dt:
            raise FletcherError(ERR_INVALID, "Copy requires matching data types (use Cast)")
        if frm.rows * frm.cols != self.rows * self.cols:
            raise FletcherError(ERR_INVALID, "Copy size mismatch")
        check(lib().fl_copy_device(self.b.ctx, self.ptr, frm.ptr,
                                   self.rows * self.cols * _esz(self.dt)))

    def Slice(self, i: int, k: int, j: int, l: int) -> "RocmTensor":
        if i < 0 or k > self.rows or j < 0 or l > self.cols or i >= k or j >= l:
            raise FletcherError(ERR_INVALID, "Invalid slice bounds")
        if j == 0 and l == self.cols:
            # Whole rows: a view at a byte offset into this tensor.
            return RocmTensor(self.b, self.ptr + i * self.cols * _esz(self.dt), k - i, self.cols,
                              self.dt, self.trans, False)
        out = self.b._result(k - i, l - j, self.dt)
        check(lib().fl_slice(self.b.ctx, self.dt, self.ptr, self.rows, self.cols, i, k, j, l,
                             out.ptr))
        return out

    def Cast(self, dt: int) -> "RocmTensor":
        out = self.b._result(self.rows, self.cols, dt)
        check(lib().fl_cast(self.b.ctx, self.ptr, self.dt, out.ptr, dt, self.rows * self.cols))
        return out

    def _as(self, dt: int):
        """(tensor in dt, temporary to put back or None)."""
        if self.dt == dt:
            return self, None
        c = self.Cast(dt)
        return c, c

    # -- ops ------------------------------------------------------------------
    def Mul(self, a: "RocmTensor", b: "RocmTensor"):
        """receiver = a * b in the receiver's type (device.go:39-42)."""
        A, ta = a._as(self.dt)
        B, tb = b._as(self.dt)
        m, k = A.Dims()
        k2, n = B.Dims()
        if k != k2 or (m, n) != self.Dims():
            raise FletcherError(ERR_INVALID, f"Dimension mismatch: {m}x{k} * {k2}x{n}")
        check(lib().fl_gemm(self.b.ctx, self.dt, int(A.trans), int(B.trans), m, n, k, 1.0, A.ptr,
                            A.cols, B.ptr, B.cols, self.ptr, self.cols))
        for t in (ta, tb):
            if t is not None:
                self.b.PutTensor(t)

    def LinearActivation(self, x: "RocmTensor", w: "RocmTensor", bias, act: int) -> "RocmTensor":
        if x.trans:
            raise FletcherError(ERR_INVALID, "Linear on a transposed input")
        r, k = x.Dims()
        k2, n = w.Dims()
        if k != k2:
            raise FletcherError(ERR_INVALID, "Linear dimension mismatch")
        bt, tmp = (None, None) if bias is None else bias._as(w.dt)
        out = self.b._result(r, n // 2 if act == ACT_SWIGLU else n, w.dt)
        # A transposed [out, in] weight is the FL_W_OUT_IN layout.
        check(lib().fl_linear(self.b.ctx, x.dt, x.ptr, r, k, w.dt, w.ptr,
                              W_OUT_IN if w.trans else W_IN_OUT, n,
                              bt.ptr if bt is not None else None, act, self.b.math, out.ptr))
        if tmp is not None:
            self.b.PutTensor(tmp)
        return out

    def Linear(self, x, w, bias) -> "RocmTensor":
        return self.LinearActivation(x, w, bias, ACT_IDENTITY)

    def Add(self, o: "RocmTensor"):
        check(lib().fl_add(self.b.ctx, self.dt, self.ptr, o.dt, o.ptr, self.rows * self.cols))

    def AddScalar(self, v: float):
        check(lib().fl_add_scalar(self.b.ctx, self.dt, self.ptr, self.rows * self.cols, v))

    def Scale(self, v: float):
        check(lib().fl_scale(self.b.ctx, self.dt, self.ptr, self.rows * self.cols, v))

    def AddBias(self, bias: "RocmTensor"):
        bt, tmp = bias._as(self.dt)
        check(lib().fl_add_bias(self.b.ctx, self.dt, self.ptr, self.rows, self.cols, bt.ptr))
        if tmp is not None:
            self.b.PutTensor(tmp)

    def _act(self, act: int):
        check(lib().fl_activation(self.b.ctx, self.dt, self.ptr, self.rows, self.cols, act,
                                  self.b.math))

    def Softmax(self):
        self._act(ACT_SOFTMAX)

    def Gelu(self):
        self._act(ACT_GELU)

    def Tanh(self):
        self._act(ACT_TANH)

    def LayerNorm(self, g: "RocmTensor", b: "RocmTensor", eps: float):
        G, tg = g._as(F32)
        B, tb = b._as(F32)
        check(lib().fl_layernorm(self.b.ctx, self.dt, self.ptr, self.rows, self.cols, G.ptr,
                                 B.ptr, eps))
        for t in (tg, tb):
            if t is not None:
                self.b.PutTensor(t)

    def AddLayerNorm(self, res: "RocmTensor", g: "RocmTensor", b: "RocmTensor", eps: float):
        G, tg = g._as(F32)
        B, tb = b._as(F32)
        check(lib().fl_add_layernorm(self.b.ctx, self.dt, self.ptr, res.dt, res.ptr, self.rows,
                                     self.cols, G.ptr, B.ptr, eps))
        for t in (tg, tb):
            if t is not None:
                self.b.PutTensor(t)

    def Gather(self, idx) -> "RocmTensor":
        i64 = np.ascontiguousarray(idx, np.int64)
        out = self.b._result(i64.size, self.cols, self.dt)
        check(lib().fl_gather_rows(self.b.ctx, self.dt, self.ptr, self.rows, self.cols,
                                   i64.ctypes.data, i64.size, out.ptr))
        return out

    def ApplyRoPE(self, batch: int, seq: int, heads: int, hd: int):
        check(lib().fl_rope(self.b.ctx, self.dt, self.ptr, batch, seq, heads, hd,
                            self.b.rope_base))

    def Attention(self, q, k, v, batch: int, seq: int, heads: int, scale: float) -> "RocmTensor":
        out = self.b._result(q.rows, q.cols, q.dt)
        check(lib().fl_attention(self.b.ctx, q.dt, q.ptr, k.ptr, v.ptr, out.ptr, batch, seq,
                                 heads, q.cols, scale, self.b.math))
        return out

    def AttentionVarLen(self, q, k, v, lengths, heads: int, scale: float) -> "RocmTensor":
        out = self.b._result(q.rows, q.cols, q.dt)
        l64 = np.ascontiguousarray(lengths, np.int64)
        check(lib().fl_attention_varlen(self.b.ctx, q.dt, q.ptr, k.ptr, v.ptr, out.ptr,
                                        l64.ctypes.data, l64.size, heads, q.cols, scale,
                                        self.b.math))
        return out

    # -- BASELINE's pooling (not a device.Tensor method) -----------------------
    def MeanPool(self, lengths, pool: int) -> "RocmTensor":
        """Masked mean (+L2 for POOL_MEAN_L2) of each sequence's rows, fp32."""
        l64 = np.ascontiguousarray(lengths, np.int64)
        out = self.b._result(l64.size, self.cols, F32)
        check(lib().fl_mean_pool(self.b.ctx, self.dt, self.ptr, self.cols, l64.ctypes.data,
                                 l64.size, int(pool == POOL_MEAN_L2), out.ptr))
        return out


def sqrt_scale(scale: float) -> float:
    """float32(math.Sqrt(float64(scale))) (bert.go:686)."""
    return float(np.float32(_math.sqrt(float(np.float32(scale)))))
